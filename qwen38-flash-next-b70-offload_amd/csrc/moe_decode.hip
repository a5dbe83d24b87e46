// Decode-size routed-expert MoE (pair mode: one row per (token, expert) pair), EXL3 trellis dequantization fused into
// the expert GEMVs, for CDNA4. One launch per MoE layer (moe_layer_kernel), two kinds of workgroups:
//
//   gate/up WGs (ids 0 .. n_gu-1), one per (pair, projection, PLANAR4 group of 4 tile-columns = 64 columns of I,
//     1024-row slice of H): issue their trellis-word loads first, then the input Hadamard of x*suh (one 128-row block
//     per wave), the trellis GEMV (one period per lane: bfe + mul + sad per weight, one v_dot2_f32_f16 per two) with an
//     in-WG reduction, and publish the 64 column sums (fp32) of the slice for the pair.
//   down WGs (ids n_gu ..), one per (pair, 128-column block of H) over the whole K = I: issue their word loads, wait
//     (bounded) for the pair's gate/up sums, run the gate/up epilogue of the pair themselves (output Hadamards * svh,
//     SiLU(g)*u, *suh_d, down-input Hadamard -> the down input in LDS, fp16), GEMV with an in-WG reduction, epilogue
//     (output Hadamard * w * svh_d) -> y (fp32). The WG of the last pick of a row (the combiner of that row and block)
//     loads the other picks' y with its wave 0 alone (no LDS round, no barrier) and sums the top-k y's in k order into
//     out; in the combiner of the last (row, block) the other waves meanwhile check that every other gate/up and down
//     workgroup has consumed its inputs (each raises a started word once it has), then wave 0 commits the
//     expert-cache fills (ptrs[e] = fill[e]; fill[e] = 0) and advances the call epoch.
// Every value handed from one workgroup to another is a tagged word (tag = call epoch + 1 in the high half, the fp32
// value in the low half) written with one 64-bit agent-scope store into a library-owned zeroed buffer: a consumer polls
// the data itself, so no producer waits for its stores and no counter is shared (same-address atomics serialize at
// the coherence point). A consumer polls the data words themselves (the gate/up sums: 4 ksn words per lane and round).
// Gate/up WGs have lower ids, so on every XCD they are dispatched before any down WG and never wait: the down WGs'
// wait always ends (it is also bounded, with an error flag, so a broken assumption cannot hang the GPU).
//
// Reference semantics: kernels/moe-a8/exl3_moe.a8.sycl GateUpKernel (121-260), DownKernel (264-368), CombineKernel
// (371-395); kernels/moe-a8/exl3_esimd.h ReconstructKernel (869-936). Accumulation is fp32 throughout (the reference
// keeps fp16 partials per tile-row); the fp16 rounding points of the epilogues are the reference's.
//
// The codebook affine w = c1*h + c2 is applied to the dot product: sum_k w_k x_k = c1 sum_k h_k x_k + c2 sum_k x_k,
// with h the exact fp16 1024 + bytesum, so the inner loop is bfe, mul and sad per weight and one v_dot2_f32_f16 per
// two weights (the two h of a dot product packed by v_sad_hi_u8).
#include "exl3_common.cuh"
#include "exl3_gemv.cuh"
#include "exl3_ensure.cuh"
#include "exl3_geom.h"
#include "exl3_kernels.h"

namespace exl3 {

__device__ unsigned g_epoch;                 // call epoch (advanced by the last workgroup of each call; never ~0u)

__device__ int g_cnt_all[4];          // [1] victim reads done, [2] fused ensure done
// [0]: bounded waits that timed out since load (0 in a healthy run). 16-byte aligned: the host tier step copies the
// four words into its pinned snapshot with 16-byte accesses.
__device__ __align__(16) int g_status[4];
// optional mirror of g_status[0] in pinned host memory (null: none), raised with a system-scope atomic by the wave
// whose wait timed out, so that a host caller can notice a timeout by reading host memory, without a copy or a sync
__device__ int* g_status_host;

constexpr int kSpinMax = 1 << 22;
constexpr uint64_t kDownLoadDelay = 200;         // 2 us in s_memrealtime ticks

// tagged exchange words: (tag << 32) | fp32 bits, one single-copy-atomic 64-bit agent-scope access
__device__ __forceinline__ void st_tag(uint64_t* p, unsigned tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// the same store for a consumer on this workgroup's XCD: workgroups are dispatched to the XCDs round-robin by
// blockIdx (i % 8 with 8 XCDs, i % 4, % 2 or the one XCD in the partitioned modes), and a workgroup-scope store stops
// in the XCD's L2, where the consumer's agent-scope load finds it about 0.35 us sooner than an agent-scope store
// written through to memory. Used only where producer and consumer blockIdx differ by a multiple of 8; if that
// assumption ever failed, the consumer's bounded poll would time out and count it in the status words.
__device__ __forceinline__ void st_tag_xcd(uint64_t* p, unsigned tag, float v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ bool tag_is(uint64_t w, unsigned tag) { return (unsigned)(w >> 32) == tag; }
__device__ __forceinline__ float tag_val(uint64_t w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ unsigned call_tag() {
    return __hip_atomic_load(&g_epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}
// bounded-spin bookkeeping shared by the polls: true once the budget is spent (counted in g_status[0])
__device__ __forceinline__ void count_timeout() {
    atomicAdd(&g_status[0], 1);
    int* h = g_status_host;
    if (h) __hip_atomic_fetch_add(h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool spin_out(int& it) {
    if (++it > kSpinMax) {
        if (lane_id() == 0) count_timeout();
        return true;
    }
    __builtin_amdgcn_s_sleep(1);
    return false;
}

// GEMV of 4 tile-rows x 8 tile-columns (one 128-column block) per wave: load() issues the word loads (and the
// optional write-through stores), compute() decodes and accumulates each lane's column pair for every column pass.
template <int K>
struct Gemv8 {
    using GM = Geo<K>;
    static constexpr int G = GM::G, D = GM::D, V = GM::V, NTW = GM::NTW, NCP = 8 / NTW, L = 32 / V;
    static constexpr int NQ = V / 8;
    static_assert(NQ >= 1, "one value octet per period at least");

    uint32_t wd[NCP][4][D];

    __device__ __forceinline__ void load(const uint32_t* tr, int tiles_n, int r0, int col_tile0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int i = 0; i < D; ++i)
                    wd[cp][rr][i] = __builtin_nontemporal_load(as_global(tr) +
                                                               word_off<K>(r0 + rr, tiles_n, col_tile0 + cp * NTW + j, p, i));
    }

    __device__ __forceinline__ void write_through(uint32_t* trd, int tiles_n, int r0, int col_tile0) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int i = 0; i < D; ++i) trd[word_off<K>(r0 + rr, tiles_n, col_tile0 + cp * NTW + j, p, i)] = wd[cp][rr][i];
    }

    // victim write-back at this wave's word positions of chunk r0: the slot's old words to the victim's RAM copy,
    // read before the write-through replaces them (every load has returned when the stores are issued)
    __device__ __forceinline__ void copy_old(const uint32_t* slot, uint32_t* host, int tiles_n, int r0,
                                             int col_tile0) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll 1
        for (int cp = 0; cp < NCP; ++cp) {      // one column pair at a time: few registers on the miss path
            uint32_t old[4][D];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int i = 0; i < D; ++i)
                    old[rr][i] = slot[word_off<K>(r0 + rr, tiles_n, col_tile0 + cp * NTW + j, p, i)];
            wait_stores();
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int i = 0; i < D; ++i)
                    host[word_off<K>(r0 + rr, tiles_n, col_tile0 + cp * NTW + j, p, i)] = old[rr][i];
        }
    }

    // xh: activations of the 128-row block, [tile-row][8] half2; xrow0 = first tile-row of this wave in the block
    __device__ __forceinline__ void compute(int xrow0, const half2_t* xh, float (&acc)[NCP][2]) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
        const int qb = ((V * p) >> 3) & 3;
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp) {
            acc[cp][0] = 0.f;
            acc[cp][1] = 0.f;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint32_t prev = (uint32_t)__shfl((int)wd[cp][rr][D - 1], src_lane, 64);
                Period<K> P;
                P.set(wd[cp][rr], prev);
                const half2_t* xr = xh + (xrow0 + rr) * 8;
                half2_t xv[2][NQ];
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int qq = 0; qq < NQ; ++qq) xv[a][qq] = xr[4 * a + ((qb + qq) & 3)];
                accum_period<K, NQ, 0>(P, xv, acc[cp]);
            }
        }
    }

    // compute() in two parts: the raw h values of the chunk's first NR tile-rows decoded while its activations are
    // still being produced (NR * 32 values, NR * 16 half2 registers per lane), then the chunk with only their dot
    // products left
    template <int NR>
    using Decoded = half2_t[NCP][NR > 0 ? NR : 1][V / 2];
    template <int NR>
    __device__ __forceinline__ void decode(Decoded<NR>& h) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp)
#pragma unroll
            for (int rr = 0; rr < NR; ++rr) {
                const uint32_t prev = (uint32_t)__shfl((int)wd[cp][rr][D - 1], src_lane, 64);
                Period<K> P;
                P.set(wd[cp][rr], prev);
                decode_period<K, 0>(P, h[cp][rr]);
            }
    }
    template <int NR>
    __device__ __forceinline__ void compute_pre(const Decoded<NR>& h, const half2_t* xh, float (&acc)[NCP][2]) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
        const int qb = ((V * p) >> 3) & 3;
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp) {
            acc[cp][0] = 0.f;
            acc[cp][1] = 0.f;
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const half2_t* xr = xh + rr * 8;
                half2_t xv[2][NQ];
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int qq = 0; qq < NQ; ++qq) xv[a][qq] = xr[4 * a + ((qb + qq) & 3)];
                if (rr < NR) {
                    dot_period<K, NQ, 0>(h[cp][rr < NR ? rr : 0], xv, acc[cp]);
                } else {
                    const uint32_t prev = (uint32_t)__shfl((int)wd[cp][rr][D - 1], src_lane, 64);
                    Period<K> P;
                    P.set(wd[cp][rr], prev);
                    accum_period<K, NQ, 0>(P, xv, acc[cp]);
                }
            }
        }
    }

    // sum lanes sharing a column (call exactly once per pass); returns true for the lane owning the column pair and
    // sets col0 (column of h = 0 within the 128-column block; h = 1 is col0 + 8)
    __device__ __forceinline__ static bool reduce(float (&acc)[2], int cp, int& col0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int mm = 1; mm < L; mm <<= 1) {
            acc[0] += lane_xor(acc[0], mm);
            acc[1] += lane_xor(acc[1], mm);
        }
        col0 = (cp * NTW + j) * 16 + ((V * p) >> 5);
        return (p % L) == 0;
    }
};


constexpr int kWaves = 8;                    // waves per workgroup (both kinds)
constexpr int kThreads = 64 * kWaves;
constexpr int kCombPicks = 10;               // other picks' y a combiner's wave 0 loads per round

struct GateUpShared {
    half2_t xq[kWaves][64];                  // per wave: Hadamard-transformed x * suh of its 128-row block
    float ssw[kWaves];                       // their sums
};
struct DownShared {
    half2_t xd[kMaxI / 2];                   // the pair's down input (fp16), [I/2]
    // the last workgroup of a call with the ensure inside: the commit, victim and mask-rewrite inputs, loaded early
    int fin_nf, fin_nv;
    int fin_ef[kEnsMaxP];                    // filled experts
    int64_t fin_fv[kEnsMaxP];                // their new slot addresses
    int fin_wb[kEnsMaxP];                    // victims copied inline (write-back keys)
    int fin_id[kEnsMaxP];                    // rewritten id of masked pick i (-1: unchanged)
};
struct LayerShared {
    union {
        GateUpShared gu;
        DownShared dn;
    } u;
    float red[kWaves][128];  // per-wave column sums
    int64_t fdst;            // write-through target of the pair (0: none)
    int fwb;                 // victims copied inline: write-back owner of that slot's old bytes (-1: none)
    int64_t fwa;             // its write-back target (the owner's RAM record)
    int last;
};

// bounded wait until *c >= target (one lane); a timeout is counted in g_status[0] and returns false
__device__ __forceinline__ bool wait_count(const int* c, int target) {
    int it = 0;
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > kSpinMax) {
            count_timeout();
            return false;
        }
    }
    return true;
}

// victim write-back (VictimCopyKernel, a8:1168-1189): workgroup (victim i, 64 KiB chunk c) copies its chunk of the
// victim's slot to the old owner's RAM-tier address and flags the owner RAM-resident. The chunk is read into registers
// first; once every load has returned the workgroup counts itself (g_cnt_all[1]), so the write-through of a miss into
// the reassigned slot can start while the copy's stores to host memory are still in flight. With the ensure inside
// the launch, the victim list is read after the ensure workgroup raised its flag.
constexpr int kVictChunk = kVictimChunkBytes;
constexpr int kVictPer = kVictChunk / 16 / kThreads;    // 16-byte words per thread
__device__ __forceinline__ void victim_wg(const DecodeArgs& A, int blk) {
    const VictimArgs& V = A.va;
    const int i = blk / A.vict_chunks, c = blk % A.vict_chunks;
    if (A.fused) {
        if (threadIdx.x == 0) wait_count(&g_cnt_all[2], 1);
        __syncthreads();
    }
    const int nv = A.fused ? ld_agent_i32(V.vict) : V.vict[0];
    const uint4* src = nullptr;
    uint4* dst = nullptr;
    int64_t q0 = 0, q1 = 0;
    if (i < nv) {
        const int old = A.fused ? ld_agent_i32(V.vict + 1 + 2 * i) : V.vict[1 + 2 * i];
        const int s = A.fused ? ld_agent_i32(V.vict + 2 + 2 * i) : V.vict[2 + 2 * i];
        if (old >= 0) {
            if (V.ram_res && c == 0 && threadIdx.x == 0) V.ram_res[old] = 1;
            src = (const uint4*)(V.slot_base + (int64_t)s * V.blob);
            dst = (uint4*)(V.vaddr ? (A.fused ? ld_agent_i64(V.vaddr + i) : V.vaddr[i])
                                   : V.host_base[old / V.E] + (int64_t)(old % V.E) * V.hstride);
            q0 = (int64_t)c * (kVictChunk >> 4);
            q1 = min(V.blob >> 4, q0 + (kVictChunk >> 4));
        }
    }
    uint4 v[kVictPer];
#pragma unroll
    for (int k = 0; k < kVictPer; ++k) {
        const int64_t q = q0 + threadIdx.x + (int64_t)k * kThreads;
        v[k] = q < q1 ? src[q] : uint4{0u, 0u, 0u, 0u};
    }
    wait_stores();                               // vmcnt(0): every load of the old bytes has returned
    __syncthreads();
    if (threadIdx.x == 0) counter_add(&g_cnt_all[1], 1);
#pragma unroll
    for (int k = 0; k < kVictPer; ++k) {
        const int64_t q = q0 + threadIdx.x + (int64_t)k * kThreads;
        if (q < q1) dst[q] = v[k];
    }
}

// pointer of the blob of pair a: precomputed by the cache's ensure (pair_ptr) or looked up through ids/ptrs
__device__ __forceinline__ const uint8_t* pair_base(const DecodeArgs& A, int a, int& e) {
    e = min(max(A.ids[a], 0), A.E - 1);          // out-of-range ids are clamped, never dereferenced
    return A.pair_ptr ? (const uint8_t*)A.pair_ptr[a] : (const uint8_t*)A.ptrs[e];
}

// Victims copied inline (slots at the blob size: a victim and the expert that replaces it share one layout): the one
// writer of each miss (the first pick of its expert) copies the victim's old bytes at exactly the positions it is
// about to overwrite to the victim's RAM copy (the reference's VictimCopyKernel a8:1168-1189, split over the
// writers); the last workgroup flags the victims RAM-resident. Returns the write-back owner of the slot at f, or -1,
// and in wa its write-back target: the record the ensure chose, or the owner's fixed record.
__device__ __forceinline__ int inline_victim(const DecodeArgs& A, int64_t f, int64_t& wa) {
    const int32_t* vl = A.va.vict;               // fields read once: the loop below has only loads
    const int s = (int)((f - A.va.slot_base) / A.va.blob);
    const int nv = ld_agent_i32(vl);
    for (int i = 0; i < nv; ++i)
        if (ld_agent_i32(vl + 2 + 2 * i) == s) {
            const int wb = ld_agent_i32(vl + 1 + 2 * i);
            if (wb >= 0)
                wa = A.va.vaddr ? ld_agent_i64(A.va.vaddr + i)
                                : A.va.host_base[wb / A.va.E] + (int64_t)(wb % A.va.E) * A.va.hstride;
            return wb;
        }
    return -1;
}

// the same with the ensure running inside the launch: the pair applies the tier mask itself (expert in neither HBM
// nor RAM -> the layer's safe expert, weight 0). Neither input changes during the call for a masked key (the ensure
// never gives it a slot; write-back victims are slot owners, never picks), and a key the ensure turns from miss into
// fill keeps ram_res = 1, so the pair and the ensure agree. ptrs[e] of every pick stays as it was at the start until
// the last workgroup commits the fills, so a pointer outside the slot arena marks a miss (a host copy).
__device__ __forceinline__ const uint8_t* pair_lookup(const DecodeArgs& A, int a, int& e, bool& miss, bool& masked) {
    const EnsureArgs& Q = A.ens;
    int id = min(max(A.ids[a], 0), A.E - 1);
    const int kb = Q.layer * A.E;
    int64_t p = A.ptrs[id];
    masked = false;
    if (Q.ram_res) {
        const int safe = Q.safe[Q.layer];
        const uint8_t rr = Q.ram_res[kb + id];
        const int so = Q.slot_of[kb + id];
        masked = !rr && so < 0;
        int sf = safe;
        asm volatile("" : "+v"(sf));             // the safe id loaded beside the mask inputs, not after them
        if (masked) {                            // (uniform) the safe expert's pointer only when it is needed: an
            id = sf;                             // unmasked pair's lookup is two rounds of loads, not three
            p = A.ptrs[sf];
        }
    }
    e = id;
    miss = p < Q.slot_base || p >= Q.slot_base + (int64_t)Q.S * Q.blob;
    return (const uint8_t*)p;
}

// gate/up WG per (pair, projection, PLANAR4 group cg of 4 tile-columns, 1024-row slice ks of H): wave w covers the
// 128-row block hb = 8 ks + w (8 tile-rows x 4 tile-columns) and its input Hadamard; waves past the end of H add 0.
template <int K>
__device__ __forceinline__ void gateup_wg(const DecodeArgs& A, int blk, LayerShared& S) {
    using GQ = Gemv4<K>;
    // issue priority over the down waves that share the CU: their weights are decoded ahead of their input, in the
    // cycles the gate/up waves (the critical path) leave free
    __builtin_amdgcn_s_setprio(2);
    const int H = A.g.H, I = A.g.I;
    const int nhb = H / 128, ksn = gu_kslices(H), ncg = I / 64;
    const int per = 2 * ncg * ksn;               // gate/up workgroups per pair
    const int a = blk / per, r = blk % per;
    const int ks = r % ksn, cg = (r / ksn) % ncg, pj = r / (ksn * ncg);
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    int e;
    bool miss = false, masked = false;
    const uint8_t* base = A.fused ? pair_lookup(A, a, e, miss, masked) : pair_base(A, a, e);
    const int m = a / A.topk;
    uint8_t* dst = !A.fused && A.fill ? (uint8_t*)A.fill[e] : nullptr;
    const int hb = ks * 8 + wv;
    const bool live = hb < nhb;
    const int tiles_n = 2 * I / 16, ct0 = pj * (I / 16) + cg * 4, rt0 = hb * 8;
    // x and suh of this wave's block first, as raw bits (no conversion, so no load waits for another), so that its
    // input Hadamard need not wait for the weight words
    uint64_t xr = 0;
    uint32_t sr = 0;
    if (live) {
        const half_t* suh = (const half_t*)(base + (pj ? A.g.off_suh_u : A.g.off_suh_g));
        const int k0 = hb * 128 + 2 * l;
        const size_t xo = (size_t)m * A.x_stride + k0;
        xr = ld_act2_raw(A.x, A.x_dt, xo);
        sr = *(const uint32_t*)(suh + k0);       // the blob's vectors are 4-byte aligned, k0 even
    }
    GQ g;
    if (live) g.load((const uint32_t*)base, tiles_n, rt0, ct0);
    float xa0, xa1;
    act2_cvt(xr, A.x_dt, xa0, xa1);
    const half2_t sa = __builtin_bit_cast(half2_t, sr);
    const half_t sa0 = sa.x, sa1 = sa.y;
    const unsigned tag = wv == 0 ? call_tag() : 0u;
    float ssum = 0.f;
    if (live) {                                  // input Hadamard of x * suh over this wave's block
        float v0 = (float)to_half(xa0 * (float)sa0);
        float v1 = (float)to_half(xa1 * (float)sa1);
        wave_fwht128(v0, v1);
        const half_t h0 = to_half(v0 * kRsqrt128), h1 = to_half(v1 * kRsqrt128);
        S.u.gu.xq[wv][l] = half2_t{h0, h1};
        ssum = wave_sum((float)h0 + (float)h1);
    }
    if (A.fused ? miss : dst != nullptr) {       // write-through of a cache miss into its HBM slot
        if (tid == 0) {
            int64_t f = (int64_t)dst;
            if (A.fused) {                       // the target is the ensure's decision
                wait_count(&g_cnt_all[2], 1);
                f = ld_agent_i64(A.fill + e);
                if (A.vict_inline && f && !ld_agent_i32(A.ens.pair_own + a)) f = 0;   // another pick writes it
            }
            if (f && A.n_vict_wg) wait_count(&g_cnt_all[1], A.n_vict_wg);   // after the victims' old bytes were read
            S.fdst = f;
            int64_t wa = 0;
            S.fwb = f && A.vict_inline ? inline_victim(A, f, wa) : -1;
            S.fwa = wa;
        }
        __syncthreads();
        dst = (uint8_t*)S.fdst;
    }
    uint8_t* hv = dst && S.fwb >= 0 ? (uint8_t*)S.fwa : nullptr;            // the victim's RAM copy
    if (dst && r == 0) {                         // the vectors (suh, svh) after the trellis words
        const uint32_t* sv = (const uint32_t*)(base + A.g.off_suh_g);
        uint32_t* dv = (uint32_t*)(dst + A.g.off_suh_g);
        const int n = (int)((A.g.blob - A.g.off_suh_g) >> 2);
        if (hv) {                                // the victim's old vectors first, 8 words per thread and round
            uint32_t* ov = (uint32_t*)(hv + A.g.off_suh_g);
            for (int i0 = 0; i0 < n; i0 += 8 * kThreads) {
                uint32_t w8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = i0 + j * kThreads + tid;
                    w8[j] = i < n ? dv[i] : 0u;
                }
                wait_stores();
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = i0 + j * kThreads + tid;
                    if (i < n) {
                        ov[i] = w8[j];
                        dv[i] = sv[i];
                    }
                }
            }
        } else {
            for (int i = tid; i < n; i += kThreads) dv[i] = sv[i];
        }
    }
    float acc[GQ::NCQ][2];
#pragma unroll
    for (int q = 0; q < GQ::NCQ; ++q) acc[q][0] = acc[q][1] = 0.f;
    if (live) {
        if (hv) g.copy_old((const uint32_t*)dst, (uint32_t*)hv, tiles_n, rt0, ct0);
        if (dst) g.write_through((uint32_t*)dst, tiles_n, rt0, ct0);
        g.compute(&S.u.gu.xq[wv][0], acc);       // the wave's own LDS rows: no barrier
    }
    if (!live) S.red[wv][l] = 0.f;
#pragma unroll
    for (int q = 0; q < GQ::NCQ; ++q) {
        int c0;
        if (GQ::reduce(acc[q], q, c0) && live) {
            S.red[wv][c0] = acc[q][0];
            S.red[wv][c0 + 8] = acc[q][1];
        }
    }
    if (l == 0) S.u.gu.ssw[wv] = ssum;
    __syncthreads();
    if (wv != 0) return;
    float t = 0.f, xs = 0.f;                     // column l of the group: the eight blocks in order
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        t += S.red[w][l];
        xs += S.u.gu.ssw[w];
    }
    st_tag(A.xpart + ((size_t)a * ksn + ks) * 2 * I + pj * I + cg * 64 + l, tag, kC1 * t + kC2 * xs);
    if (l == 0) st_tag(A.xstart + blk, tag, 0.f);    // its inputs (ids, pointers, fill target) are consumed
}

// down WG per (pair, 128-column block of H) over the full K = I: the 4-row chunks of the I/16 tile-rows go round-robin
// to the eight waves, the per-wave column sums are reduced in LDS in wave order (no cross-WG exchange), then the output
// Hadamard * w * svh_d -> y, and the combine.
// NR > 0: every wave has at most one 4-row chunk (I <= 512), whose first NR tile-rows are decoded ahead of the down
// input, and no second chunk's words are held across the wait
template <int K, int NR>
__device__ __forceinline__ void down_wg(const DecodeArgs& A, int blk, LayerShared& S) {
    using GV = Gemv8<K>;
    const int H = A.g.H, I = A.g.I;
    const int nbn = H / 128, kt = I / 16;
    const int nb = blk % nbn, a = blk / nbn;
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    int e;
    bool miss = false, masked = false;
    const uint8_t* base = A.fused ? pair_lookup(A, a, e, miss, masked) : pair_base(A, a, e);
    const int m = a / A.topk;
    const int tiles_n = H / 16, ct0 = nb * 8;
    const uint32_t* tr = (const uint32_t*)(base + A.g.gu_bytes);
    const int nch0 = (kt / 4 + kWaves - 1 - wv) / kWaves;     // 4-row chunks of this wave: q = wv + kWaves * c
    const int nch = NR > 0 ? min(nch0, 1) : nch0;
    {   // the down weights are needed only after the gate/up phase: let the gate/up loads (the critical path) take
        // HBM first, then issue these (constant 100 MHz clock)
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__builtin_amdgcn_s_memrealtime() - t0 < kDownLoadDelay) __builtin_amdgcn_s_sleep(4);
    }
    GV g0, g1;
    if (nch > 0) g0.load(tr, tiles_n, wv * 4, ct0);
    if (nch > 1) g1.load(tr, tiles_n, (wv + kWaves) * 4, ct0);
    half2_t sc_d{};                              // epilogue scale and routing weight (wave 0), loaded early
    float wgt = 0.f;
    if (wv == 0) {
        sc_d = *(const half2_t*)((const half_t*)(base + A.g.off_svh_d) + nb * 128 + 2 * l);
        wgt = masked ? 0.f : A.w[a];
    }
    half2_t e_g{}, e_u{}, e_d{};                 // gate/up epilogue scales of this wave's first 128-column block of I
    if (wv < I / 128) {
        const int cI = wv * 128 + 2 * l;
        e_g = *(const half2_t*)((const half_t*)(base + A.g.off_svh_g) + cI);
        e_u = *(const half2_t*)((const half_t*)(base + A.g.off_svh_u) + cI);
        e_d = *(const half2_t*)((const half_t*)(base + A.g.off_suh_d) + cI);
    }
    const unsigned tag = call_tag();
    if (A.fused && a == A.npairs - 1 && nb == nbn - 1 && wv == kWaves - 1) {
        // the last workgroup of the call (it combines the last row and block): once the ensure's decisions are final,
        // load what the end of the call stores, so that the end has no dependent loads left (at most kEnsMaxP picks)
        if (l == 0) wait_count(&g_cnt_all[2], 1);
        const int nf = A.commit_ptrs ? ld_agent_i32(A.fill_list) : 0;
        const int nvv = A.vict_inline && A.va.ram_res ? ld_agent_i32(A.va.vict) : 0;
        int ef = -1, wb = -1, nid = -1;
        int64_t fv = 0;
        if (l < nf) {
            ef = ld_agent_i32(A.fill_list + 1 + l);
            fv = ld_agent_i64(A.commit_fill + ef);
        }
        if (l < nvv) wb = ld_agent_i32(A.va.vict + 1 + 2 * l);
        const EnsureArgs& Q = A.ens;
        if (Q.ram_res && l < A.npairs) {         // the mask rule gives the same answer as at the pairs' start
            const int kb = Q.layer * A.E, id = min(max(Q.ids[l], 0), A.E - 1);
            if (!Q.ram_res[kb + id] && Q.slot_of[kb + id] < 0) nid = Q.safe[Q.layer];
        }
        S.u.dn.fin_ef[l] = ef;
        S.u.dn.fin_fv[l] = fv;
        S.u.dn.fin_wb[l] = wb;
        S.u.dn.fin_id[l] = nid;
        if (l == 0) {
            S.u.dn.fin_nf = nf;
            S.u.dn.fin_nv = nvv;
        }
    }
    if (tid == 0) {                              // write-through target of a miss
        int64_t f = !A.fused && A.fill ? A.fill[e] : 0;
        if (A.fused && miss) {                   // the write-through target is the ensure's decision
            wait_count(&g_cnt_all[2], 1);
            f = ld_agent_i64(A.fill + e);
            if (A.vict_inline && f && !ld_agent_i32(A.ens.pair_own + a)) f = 0;       // another pick writes it
        }
        if (f && A.n_vict_wg) wait_count(&g_cnt_all[1], A.n_vict_wg);      // and for the victims' old bytes
        S.fdst = f;
        int64_t wa = 0;
        S.fwb = f && A.vict_inline ? inline_victim(A, f, wa) : -1;
        S.fwa = wa;
    }
    // with one chunk per wave, a call that can fill copies the victim's old words and writes its words through now
    // (the target is the ensure's decision, taken before these loads return), so that they are dead once decoded
    bool done_wt = false;
    if constexpr (NR > 0) {
        if (A.fused || A.fill) {
            __syncthreads();                     // the target and the victim from thread 0
            uint32_t* trd0 = S.fdst ? (uint32_t*)((uint8_t*)S.fdst + A.g.gu_bytes) : nullptr;
            if (trd0 && nch > 0) {
                if (S.fwb >= 0) g0.copy_old(trd0, (uint32_t*)((uint8_t*)S.fwa + A.g.gu_bytes), tiles_n, wv * 4, ct0);
                g0.write_through(trd0, tiles_n, wv * 4, ct0);
            }
            done_wt = true;
        }
    }
    // the first chunk's raw h values decoded now, while the gate/up sums are still being produced: only its dot
    // products are left once the down input is known (the asm keeps the decode ahead of the wait)
    typename GV::template Decoded<NR> hd;
    if (NR > 0 && nch > 0) {
        g0.template decode<NR>(hd);
#pragma unroll
        for (int cp = 0; cp < GV::NCP; ++cp)
#pragma unroll
            for (int rr = 0; rr < NR; ++rr)
#pragma unroll
                for (int i = 0; i < GV::V / 2; ++i) {
                    uint32_t b = __builtin_bit_cast(uint32_t, hd[cp][rr][i]);
                    asm volatile("" : "+v"(b));
                    hd[cp][rr][i] = __builtin_bit_cast(half2_t, b);
                }
    }
    const int ksn = gu_kslices(H);
    half2_t* xs = S.u.dn.xd;                     // the pair's down input, [I/2] half2
    // gate/up epilogue of the pair, one 128-column block b of I per wave and round: wait for the sums of its 4 * ksn
    // gate/up workgroups (gate and up, column groups 2b and 2b + 1, every K-slice), then output Hadamards * svh,
    // SiLU(g)*u, * suh_d, down-input Hadamard (the reference's fp16 rounding points)
    {
        const uint64_t* pg = A.xpart + (size_t)a * ksn * 2 * I;
        for (int b = wv; b < I / 128; b += kWaves) {
            const int cI = b * 128 + 2 * l;
            float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
            for (int k0 = 0; k0 < ksn; k0 += 2) {        // the K-slices in order, two at a time
                uint64_t v[2][4];
                int it = 0;
                for (;;) {                   // all eight loads in flight (no branch), then the tag checks
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const uint64_t* q = pg + (size_t)min(k0 + k, ksn - 1) * 2 * I + cI;
                        v[k][0] = ld_tag(q);
                        v[k][1] = ld_tag(q + 1);
                        v[k][2] = ld_tag(q + I);
                        v[k][3] = ld_tag(q + I + 1);
                    }
                    bool ok = true;
#pragma unroll
                    for (int k = 0; k < 2; ++k)
#pragma unroll
                        for (int i = 0; i < 4; ++i) ok &= (k0 + k >= ksn) | tag_is(v[k][i], tag);
                    if (__all(ok) || spin_out(it)) break;
                }
#pragma unroll
                for (int k = 0; k < 2; ++k)
                    if (k0 + k < ksn) {
                        g0 += tag_val(v[k][0]);
                        g1 += tag_val(v[k][1]);
                        u0 += tag_val(v[k][2]);
                        u1 += tag_val(v[k][3]);
                    }
            }
            if (b != wv) {
                e_g = *(const half2_t*)((const half_t*)(base + A.g.off_svh_g) + cI);
                e_u = *(const half2_t*)((const half_t*)(base + A.g.off_svh_u) + cI);
                e_d = *(const half2_t*)((const half_t*)(base + A.g.off_suh_d) + cI);
            }
            wave_fwht128(g0, g1);
            wave_fwht128(u0, u1);
            g0 = (float)to_half(g0 * kRsqrt128 * (float)e_g.x);
            g1 = (float)to_half(g1 * kRsqrt128 * (float)e_g.y);
            u0 = (float)to_half(u0 * kRsqrt128 * (float)e_u.x);
            u1 = (float)to_half(u1 * kRsqrt128 * (float)e_u.y);
            float a0 = (float)to_half(silu_mul(g0, u0));
            float a1 = (float)to_half(silu_mul(g1, u1));
            a0 = (float)to_half(a0 * (float)e_d.x);
            a1 = (float)to_half(a1 * (float)e_d.y);
            wave_fwht128(a0, a1);
            xs[b * 64 + l] = half2_t{to_half(a0 * kRsqrt128), to_half(a1 * kRsqrt128)};
        }
    }
    __syncthreads();
    if (tid == 0) st_tag(A.xstart + A.n_gu + blk, tag, 0.f);     // ids, pointers, w and fill target consumed
    // (no write-through target at all when the call has no fills: then the words are dead once decoded)
    uint32_t* trd = !done_wt && (A.fused || A.fill) && S.fdst ? (uint32_t*)((uint8_t*)S.fdst + A.g.gu_bytes) : nullptr;
    if (trd && S.fwb >= 0) {                     // the victim's old down words at this wave's positions, first
        uint32_t* tro = (uint32_t*)((uint8_t*)S.fwa + A.g.gu_bytes);
        for (int c = 0; c < nch; ++c) g0.copy_old(trd, tro, tiles_n, (wv + kWaves * c) * 4, ct0);
    }
    float acc[GV::NCP][2], tacc[GV::NCP][2];
    float xsum = 0.f;
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) acc[cp][0] = acc[cp][1] = 0.f;
    // chunk c is in g0 and chunk c + 1 in g1: compute g0, move g1 into g0 (it has to have arrived by now anyway),
    // then load chunk c + 2 into g1, so that every load overlaps one chunk's compute (with the buffer picked at run
    // time instead, the compiler made each prefetch wait for its own loads)
    for (int c = 0; c < nch; ++c) {
        const int r0 = (wv + kWaves * c) * 4;
        if (trd) g0.write_through(trd, tiles_n, r0, ct0);
        if (NR > 0 && c == 0) g0.template compute_pre<NR>(hd, xs + r0 * 8, tacc);
        else g0.compute(0, xs + r0 * 8, tacc);
        if (c + 1 < nch) {
            g0 = g1;
            if (c + 2 < nch) g1.load(tr, tiles_n, r0 + 8 * kWaves, ct0);
        }
#pragma unroll
        for (int cp = 0; cp < GV::NCP; ++cp) {
            acc[cp][0] += tacc[cp][0];
            acc[cp][1] += tacc[cp][1];
        }
        {   // sum of the 64 activations of these 4 tile-rows (raw-h correction)
            const half2_t v = xs[r0 * 8 + (l & 31)];
            xsum += (l < 32) ? (float)v.x + (float)v.y : 0.f;
        }
    }
    xsum = wave_sum(xsum);
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) {
        int c0;
        const bool own = GV::reduce(acc[cp], cp, c0);
        if (own) {
            S.red[wv][c0] = kC1 * acc[cp][0] + kC2 * xsum;
            S.red[wv][c0 + 8] = kC1 * acc[cp][1] + kC2 * xsum;
        }
    }
    __syncthreads();
    const int k = a % A.topk;
    const bool comb = k == A.topk - 1;           // combiner of (row m, block nb): the row's last pick, highest id
    const int nfin = A.M * nbn, me = m * nbn + nb;
    const bool fin = comb && me == nfin - 1;     // the last combiner of the call also commits
    if (wv != 0 && !fin) return;
    const int c = nb * 128 + 2 * l;
    float v0 = 0.f, v1 = 0.f;
    uint64_t* yb = A.xy + (size_t)(m * A.topk) * H + c;
    if (wv == 0) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            v0 += S.red[w][2 * l];
            v1 += S.red[w][2 * l + 1];
        }
        wave_fwht128(v0, v1);
        const float sc = kRsqrt128 * wgt;
        v0 = v0 * sc * (float)sc_d.x;
        v1 = v1 * sc * (float)sc_d.y;
        asm volatile("" : "+v"(v0), "+v"(v1));   // y rounded as stored (not fused into the combiner's sum)
        if (!comb) {                             // y of this pick for the row's combiner
            // the down workgroups of one column block nb, all picks, sit 16 a apart in blockIdx: with nbn a multiple
            // of 8 they share an XCD with their combiner
            if (nbn % 8 == 0) {
                st_tag_xcd(yb + (size_t)k * H, tag, v0);
                st_tag_xcd(yb + (size_t)k * H + 1, tag, v1);
            } else {
                st_tag(yb + (size_t)k * H, tag, v0);
                st_tag(yb + (size_t)k * H + 1, tag, v1);
            }
            return;
        }
        // combiner: wave 0 loads the other picks' y (lower workgroup ids) itself, up to kCombPicks per round, and sums
        // them in k order before its own pick's
        float o0 = 0.f, o1 = 0.f;
        for (int k0 = 0; k0 < A.topk - 1; k0 += kCombPicks) {
            uint64_t yw[kCombPicks][2];
            int it = 0;
            for (;;) {                       // all loads in flight (no branch), then the tag checks
#pragma unroll
                for (int j = 0; j < kCombPicks; ++j) {
                    const uint64_t* q = yb + (size_t)min(k0 + j, A.topk - 2) * H;
                    yw[j][0] = ld_tag(q);
                    yw[j][1] = ld_tag(q + 1);
                }
                bool ok = true;
#pragma unroll
                for (int j = 0; j < kCombPicks; ++j)
                    ok &= (k0 + j >= A.topk - 1) | (tag_is(yw[j][0], tag) & tag_is(yw[j][1], tag));
                if (__all(ok) || spin_out(it)) break;
            }
#pragma unroll
            for (int j = 0; j < kCombPicks; ++j)
                if (k0 + j < A.topk - 1) {
                    o0 += tag_val(yw[j][0]);
                    o1 += tag_val(yw[j][1]);
                }
        }
        o0 += v0;
        o1 += v1;
        const size_t oo = (size_t)m * A.out_stride + c;
        st_act(A.out, A.x_dt, oo, o0);
        st_act(A.out, A.x_dt, oo + 1, o1);
    } else {
        // the last combiner's other waves: every other workgroup has raised its started word (its inputs consumed)
        const int nstart = A.n_gu + A.npairs * nbn - 1;       // every workgroup before this one
        int it = 0;
        for (;;) {
            bool ok = true;
            for (int i = tid - 64; i < nstart; i += kThreads - 64) ok = ok && tag_is(ld_tag(A.xstart + i), tag);
            if (__all(ok) || spin_out(it)) break;
        }
    }
    if (!fin) return;
    __syncthreads();
    if (wv != 0) return;
    // the last (row, block) of the layer: every other workgroup has consumed its inputs; advance the epoch and commit
    // the cache fills
    if (l == 0) {
        // every victim workgroup has counted itself: clear for the next call. After a timed-out wait the count stays
        // (the status word is non-zero and the host tier step raises), so no later call proceeds on a partial count.
        if (A.n_vict_wg && wait_count(&g_cnt_all[1], A.n_vict_wg)) counter_reset(&g_cnt_all[1]);
        const unsigned ep = tag == ~0u ? 0u : tag;   // the next call's tag is never 0 (the zeroed buffer)
        __hip_atomic_store(&g_epoch, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (A.fused) {                               // stores only: the inputs were loaded at the workgroup's start
        // every writer has copied its part: the victims' RAM copies are valid
        if (l < S.u.dn.fin_nv && S.u.dn.fin_wb[l] >= 0) A.va.ram_res[S.u.dn.fin_wb[l]] = 1;
        // the ensure's in-place rewrite of the caller's picks (masked -> safe expert, weight 0), deferred to here
        // because every pair read them during the call
        if (l < A.npairs && S.u.dn.fin_id[l] >= 0) {
            A.ens.ids[l] = S.u.dn.fin_id[l];
            A.ens.w[l] = 0.f;
        }
        if (l < S.u.dn.fin_nf) {                 // commit the fills
            A.commit_ptrs[S.u.dn.fin_ef[l]] = S.u.dn.fin_fv[l];
            A.commit_fill[S.u.dn.fin_ef[l]] = 0;
        }
        if (l == 0) counter_reset(&g_cnt_all[2]);
        return;
    }
    if (!A.commit_ptrs) return;
    const int nf = A.fill_list[0];
    for (int i = l; i < nf; i += 64) {
        const int ef = A.fill_list[1 + i];
        A.commit_ptrs[ef] = A.commit_fill[ef];
        A.commit_fill[ef] = 0;
    }
}

// MODE 1: the plain resident call (no cache: no ensure, victims, write-through, commit or precomputed pair pointers),
// compiled without those paths (21.6 KB of code against 54.6 KB for K = 3, no SGPR spills); MODE 2: the tier's cached
// call (ensure inside the launch, victims copied inline by the writers of each miss, no victim workgroups); MODE 0:
// every other combination. Each instantiation carries only its own paths, so the hot code of a call stays small.
// ONE: I <= 512, the down waves decode the weights of their one chunk (all four tile-rows) ahead of their input,
// within 128 VGPRs: 4 waves per SIMD, so a gate/up and a down workgroup share a CU. The lean call is held to 128 VGPRs for wider I too (K = 4 needs 148
// otherwise, one workgroup per CU; at 128 it spills 5, and runs the H 4096 / I 1536 layer in 38.0 us against 48.2).
template <int K, int MODE, bool ONE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(ONE || MODE == 1 ? 4 : 1)))
moe_layer_kernel(DecodeArgs A0) {
    DecodeArgs A = A0;
    if constexpr (MODE == 1) {       // lean
        A.fused = 0;
        A.fill = nullptr;
        A.pair_ptr = nullptr;
        A.commit_ptrs = nullptr;
        A.n_vict_wg = 0;
        A.vict_inline = 0;
    } else if constexpr (MODE == 2) {   // fused ensure, victims copied inline
        A.fused = 1;
        A.pair_ptr = nullptr;
        A.n_vict_wg = 0;
        A.vict_inline = 1;
    }
    __shared__ __align__(16) uint8_t lds[sizeof(LayerShared) > sizeof(EnsureShared) ? sizeof(LayerShared)
                                                                                     : sizeof(EnsureShared)];
    LayerShared& S = *reinterpret_cast<LayerShared*>(lds);
    const int nv = A.n_vict_wg;
    const int n_gu = A.n_gu;
    int b = blockIdx.x;
    if (A.fused) {                               // workgroup 0: the cache's ensure (never waits on another workgroup)
        if (b == 0) {
            ensure_wg<kThreads>(A.ens, *reinterpret_cast<EnsureShared*>(lds), &g_cnt_all[2]);
            return;
        }
        --b;
    }
    if (b < nv) victim_wg(A, b);
    else if (b < nv + n_gu) gateup_wg<K>(A, b - nv, S);
    else down_wg<K, ONE ? 4 : 0>(A, b - nv - n_gu, S);
}

// bit-exact dequantization of one trellis matrix (PLANAR4 words [k_tiles][n_tiles][8K]) -> fp16 [16 k_tiles][16 n_tiles]
template <int K>
__global__ void __launch_bounds__(256) dequant_kernel(const uint32_t* __restrict__ tr, half_t* __restrict__ out,
                                                      int k_tiles, int n_tiles) {
    using GM = Geo<K>;
    constexpr int G = GM::G, D = GM::D, NTW = GM::NTW;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int strips = (n_tiles + NTW - 1) / NTW;
    if (wave >= k_tiles * strips) return;
    const int r = wave / strips, st = wave % strips;
    const int l = lane_id(), p = l % G, j = l / G;
    const int tile = st * NTW + j;
    const bool ok = tile < n_tiles;
    uint32_t wd[D];
#pragma unroll
    for (int i = 0; i < D; ++i) wd[i] = ok ? tr[word_off<K>(r, n_tiles, tile, p, i)] : 0u;
    const uint32_t prev = (uint32_t)__shfl((int)wd[D - 1], j * G + ((p + G - 1) % G), 64);
    if (!ok) return;
    Period<K> P;
    P.set(wd, prev);
    const size_t n_out = (size_t)n_tiles * 16;
    half_t* o = out + (size_t)r * 16 * n_out + (size_t)tile * 16;
    dequant_store<K, 0>(P, p, o, n_out);
}

// ---- host launchers ------------------------------------------------------------------------------------------------

template <int K, bool ONE>
static void launch_layer_k(int mode, dim3 grid, const DecodeArgs& a, hipStream_t s) {
    if (mode == 1) hipLaunchKernelGGL((moe_layer_kernel<K, 1, ONE>), grid, dim3(kThreads), 0, s, a);
    else if (mode == 2) hipLaunchKernelGGL((moe_layer_kernel<K, 2, ONE>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((moe_layer_kernel<K, 0, ONE>), grid, dim3(kThreads), 0, s, a);
}

hipError_t launch_moe_layer(int K, const DecodeArgs& a, hipStream_t s) {
    const int n_gu = a.n_gu;
    const int n_dn = a.npairs * (a.g.H / 128);
    dim3 grid((unsigned)(a.fused + a.n_vict_wg + n_gu + n_dn));
    const bool lean = !a.fused && !a.fill && !a.pair_ptr && !a.commit_ptrs && !a.n_vict_wg && !a.vict_inline;
    const int mode = lean ? 1 : (a.fused && !a.pair_ptr && !a.n_vict_wg && a.vict_inline ? 2 : 0);
    const bool one = a.g.I / 64 <= kWaves;       // at most one 4-row chunk per down wave
    if (K == 2) one ? launch_layer_k<2, true>(mode, grid, a, s) : launch_layer_k<2, false>(mode, grid, a, s);
    else if (K == 3) one ? launch_layer_k<3, true>(mode, grid, a, s) : launch_layer_k<3, false>(mode, grid, a, s);
    else if (K == 4) one ? launch_layer_k<4, true>(mode, grid, a, s) : launch_layer_k<4, false>(mode, grid, a, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

int read_status(int* out, hipStream_t s) {
    return (int)hipMemcpyFromSymbolAsync(out, HIP_SYMBOL(g_status), sizeof(int) * 4, 0, hipMemcpyDeviceToHost, s);
}

// device address of the status words on the current device (each device holds its own copy)
hipError_t status_address(void** p) { return hipGetSymbolAddress(p, HIP_SYMBOL(g_status)); }
hipError_t status_host_slot(void** p) { return hipGetSymbolAddress(p, HIP_SYMBOL(g_status_host)); }

// the host mirror of the timeout count on the current device (a synchronous copy of the pointer into the symbol)
hipError_t set_status_mirror(int* host_word) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_status_host), &host_word, sizeof(host_word), 0, hipMemcpyHostToDevice);
}

hipError_t launch_dequant(int K, const uint32_t* tr, _Float16* out, int k_tiles, int n_tiles, hipStream_t s) {
    int ntw = K == 3 ? Geo<3>::NTW : (K == 2 ? Geo<2>::NTW : Geo<4>::NTW);
    int waves = k_tiles * ((n_tiles + ntw - 1) / ntw);
    dim3 grid((unsigned)((waves + 3) / 4));
    if (K == 2) hipLaunchKernelGGL(dequant_kernel<2>, grid, dim3(256), 0, s, tr, out, k_tiles, n_tiles);
    else if (K == 3) hipLaunchKernelGGL(dequant_kernel<3>, grid, dim3(256), 0, s, tr, out, k_tiles, n_tiles);
    else if (K == 4) hipLaunchKernelGGL(dequant_kernel<4>, grid, dim3(256), 0, s, tr, out, k_tiles, n_tiles);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace exl3
