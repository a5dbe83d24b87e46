// Decode-size routed-expert MoE (pair mode: one row per (token, expert) pair), EXL3 trellis dequantization fused into
// the expert GEMVs, for CDNA4. One launch per MoE layer (moe_layer_kernel), two kinds of workgroups:
//
//   gate/up WGs (ids 0 .. n_gu-1), one per (pair, 128-column block of I, 256-row slice of H): issue their trellis-word
//     loads first, then the input Hadamard of x*suh for gate and up, the trellis GEMV (one period per lane: bfe + mul
//     + sad + fma_mix per weight) and split-K partials; the last-arriving WG of a (pair, block) reduces the partials in
//     fixed order and runs the epilogue (output Hadamards * svh, SiLU(g)*u, *suh_d, down-input Hadamard) -> abuf
//     (fp16) and counts the block as ready for the pair.
//   down WGs (ids n_gu ..), one per (pair, 128-column block of H) over the whole K = I: issue their word loads, wait
//     (bounded) until the pair's abuf is complete, GEMV with an in-WG reduction, epilogue (output Hadamard * w *
//     svh_d) -> y (fp32); the last pair of a (row, block) sums the top-k y's in k order into out (the combine); the
//     last (row, block) commits the expert-cache fills (ptrs[e] = fill[e]; fill[e] = 0) and clears the ready counts.
// Gate/up WGs have lower ids, so on every XCD they are dispatched before any down WG and never wait: the down WGs'
// wait always ends (it is also bounded, with an error flag, so a broken assumption cannot hang the GPU).
//
// Reference semantics: kernels/moe-a8/exl3_moe.a8.sycl GateUpKernel (121-260), DownKernel (264-368), CombineKernel
// (371-395); kernels/moe-a8/exl3_esimd.h ReconstructKernel (869-936). Accumulation is fp32 throughout (the reference
// keeps fp16 partials per tile-row); the fp16 rounding points of the epilogues are the reference's.
//
// The codebook affine w = c1*h + c2 is applied to the dot product: sum_k w_k x_k = c1 sum_k h_k x_k + c2 sum_k x_k,
// with h the exact fp16 1024 + bytesum, so the inner loop is bfe, mul, sad and one mixed-precision FMA per weight.
#include "exl3_common.cuh"
#include "exl3_ensure.cuh"
#include "exl3_geom.h"
#include "exl3_kernels.h"

namespace exl3 {

__device__ int g_cnt_gu[kMaxPairs * 64];
__device__ int g_cnt_d[kMaxPairs * 64];
__device__ int g_cnt_c[kMaxRows * 64];
__device__ int g_ready[kMaxPairs];
__device__ int g_cnt_all[4];          // [0] combines done, [1] victim reads done, [2] fused ensure done
__device__ int g_status[4];          // [0]: spin timeouts (should stay 0)

constexpr int kSpinMax = 1 << 22;
constexpr uint64_t kDownLoadDelay = 120;         // 1.2 us in s_memrealtime ticks

// one period of one tile-row: xv[a][qq] holds activation rows (8a + 2q, 8a + 2q + 1), q = (qb + qq) & 3
template <int K, int NQ, int u>
__device__ __forceinline__ void accum_period(const Period<K>& P, const half2_t (&xv)[2][NQ], float (&acc)[2]) {
    if constexpr (u < Geo<K>::V) {
        const half_t h = cb_h(P.template state<u>());
        const half2_t xp = xv[(u >> 1) & 1][u >> 3];
        const half_t xs = (u & 1) ? xp.y : xp.x;
        acc[(u >> 2) & 1] = __builtin_fmaf((float)h, (float)xs, acc[(u >> 2) & 1]);
        accum_period<K, NQ, u + 1>(P, xv, acc);
    }
}

// bit-exact store of one period's values (row/col of value u depend on the period for K != 3)
template <int K, int u>
__device__ __forceinline__ void dequant_store(const Period<K>& P, int p, _Float16* o, size_t n_out) {
    if constexpr (u < Geo<K>::V) {
        o[(size_t)val_row<K>(p, u) * n_out + val_col<K>(p, u)] = cb_w(P.template state<u>());
        dequant_store<K, u + 1>(P, p, o, n_out);
    }
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

    // sum lanes sharing a column (call exactly once per pass); returns true for the lane owning the column pair and
    // sets col0 (column of h = 0 within the 128-column block; h = 1 is col0 + 8)
    __device__ __forceinline__ static bool reduce(float (&acc)[2], int cp, int& col0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int mm = 1; mm < L; mm <<= 1) {
            acc[0] += __shfl_xor(acc[0], mm, 64);
            acc[1] += __shfl_xor(acc[1], mm, 64);
        }
        col0 = (cp * NTW + j) * 16 + ((V * p) >> 5);
        return (p % L) == 0;
    }
};

constexpr int kWaves = 8;                    // waves per workgroup (both kinds)
constexpr int kThreads = 64 * kWaves;

struct LayerShared {
    half2_t xh[2][2][64];    // gate/up WG: activations of its two 128-row blocks, [proj][block][64] half2
    float ssum[2][2];
    float red[kWaves][128];  // per-wave column sums
    float tot[256];          // reduced split-K partials of the last-arriving gate/up WG
    half2_t xd[kMaxI / 2];   // down WG: the pair's abuf
    int64_t fdst;            // write-through target of the pair (0: none)
    int last;
};

// bounded wait until *c >= target (one lane); a timeout is counted in g_status[0]
__device__ __forceinline__ void wait_count(const int* c, int target) {
    int it = 0;
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (++it > kSpinMax) {
            atomicAdd(&g_status[0], 1);
            break;
        }
    }
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
            dst = (uint4*)(V.host_base[old / V.E] + (int64_t)(old % V.E) * V.hstride);
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
        const int64_t ps = A.ptrs[safe];
        const uint8_t rr = Q.ram_res[kb + id];
        const int so = Q.slot_of[kb + id];
        masked = !rr && so < 0;
        if (masked) {
            id = safe;
            p = ps;
        }
    }
    e = id;
    miss = p < Q.slot_base || p >= Q.slot_base + (int64_t)Q.S * Q.blob;
    return (const uint8_t*)p;
}

// gate/up WG per (pair, 128-column block of I, 256-row slice of H): waves (proj = w & 1, quarter = w >> 1) each cover
// 4 tile-rows x 8 tile-columns.
template <int K>
__device__ __forceinline__ void gateup_wg(const DecodeArgs& A, int blk, LayerShared& S) {
    using GV = Gemv8<K>;
    const int H = A.g.H, I = A.g.I;
    const int nbn = I / 128, ksn = gu_slices(H);
    const int ks = blk % ksn;
    blk /= ksn;
    const int nb = blk % nbn, a = blk / nbn;
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    int e;
    bool miss = false, masked = false;
    const uint8_t* base = A.fused ? pair_lookup(A, a, e, miss, masked) : pair_base(A, a, e);
    const int m = a / A.topk;
    uint8_t* dst = !A.fused && A.fill ? (uint8_t*)A.fill[e] : nullptr;
    const int proj = wv & 1, qt = wv >> 1;
    const int tiles_n = 2 * I / 16, r0 = ks * 16 + qt * 4, ct0 = proj * (I / 16) + nb * 8;

    // the last slice of an H that is an odd multiple of 128 has one 128-row block: its second-block waves only add 0
    const bool live = ks * 256 + (qt >> 1) * 128 < H;
    GV g;
    if (live) g.load((const uint32_t*)base, tiles_n, r0, ct0);
    half2_t sc_g{}, sc_u{}, sc_d{};              // epilogue scales (wave 0), loaded early: off the critical path
    if (wv == 0) {
        const int c = nb * 128 + 2 * l;
        sc_g = *(const half2_t*)((const half_t*)(base + A.g.off_svh_g) + c);
        sc_u = *(const half2_t*)((const half_t*)(base + A.g.off_svh_u) + c);
        sc_d = *(const half2_t*)((const half_t*)(base + A.g.off_suh_d) + c);
    }
    if (wv < 4 && ks * 256 + (wv >> 1) * 128 >= H) {
        if (l == 0) S.ssum[wv & 1][wv >> 1] = 0.f;
    } else if (wv < 4) {                         // input Hadamards of x * suh: (proj, 128-row block) per wave
        const int pj = wv & 1, hb = wv >> 1;
        const half_t* suh = (const half_t*)(base + (pj ? A.g.off_suh_u : A.g.off_suh_g));
        const int k0 = ks * 256 + hb * 128 + 2 * l;
        const size_t xo = (size_t)m * A.x_stride + k0;
        float v0 = (float)(half_t)(ld_act(A.x, A.x_dt, xo) * (float)suh[k0]);
        float v1 = (float)(half_t)(ld_act(A.x, A.x_dt, xo + 1) * (float)suh[k0 + 1]);
        wave_fwht128(v0, v1);
        const half_t h0 = (half_t)(v0 * kRsqrt128), h1 = (half_t)(v1 * kRsqrt128);
        S.xh[pj][hb][l] = half2_t{h0, h1};
        const float s = wave_sum((float)h0 + (float)h1);
        if (l == 0) S.ssum[pj][hb] = s;
    }
    if (A.fused ? miss : dst != nullptr) {       // write-through of a cache miss into its HBM slot
        if (tid == 0) {
            int64_t f = (int64_t)dst;
            if (A.fused) {                       // the target is the ensure's decision
                wait_count(&g_cnt_all[2], 1);
                f = ld_agent_i64(A.fill + e);
            }
            if (f && A.n_vict_wg) wait_count(&g_cnt_all[1], A.n_vict_wg);   // after the victims' old bytes were read
            S.fdst = f;
        }
        __syncthreads();
        dst = (uint8_t*)S.fdst;
    }
    if (dst) {
        if (live) g.write_through((uint32_t*)dst, tiles_n, r0, ct0);
        if (nb == 0 && ks == 0) {
            const uint32_t* sv = (const uint32_t*)(base + A.g.off_suh_g);
            uint32_t* dv = (uint32_t*)(dst + A.g.off_suh_g);
            const int n = (int)((A.g.blob - A.g.off_suh_g) >> 2);
            for (int i = tid; i < n; i += kThreads) dv[i] = sv[i];
        }
    }
    __syncthreads();
    float acc[GV::NCP][2];
    if (live) {
        g.compute((qt & 1) * 4, &S.xh[proj][qt >> 1][0], acc);
    } else {
#pragma unroll
        for (int cp = 0; cp < GV::NCP; ++cp) acc[cp][0] = acc[cp][1] = 0.f;
    }
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) {
        int c0;
        if (GV::reduce(acc[cp], cp, c0)) {
            S.red[wv][c0] = acc[cp][0];
            S.red[wv][c0 + 8] = acc[cp][1];
        }
    }
    __syncthreads();
    if (tid < 256) {                             // column tid of [gate 128 | up 128]: sum the 4 quarters in order
        const int pj = tid >> 7, c = tid & 127;
        const float t = S.red[pj][c] + S.red[pj + 2][c] + S.red[pj + 4][c] + S.red[pj + 6][c];
        st_agent(A.part_gu + ((size_t)(a * nbn + nb) * ksn + ks) * 256 + tid,
                 kC1 * t + kC2 * (S.ssum[pj][0] + S.ssum[pj][1]));
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) S.last = counter_add(&g_cnt_gu[a * nbn + nb], 1) == ksn - 1;
    __syncthreads();
    if (!S.last) return;
    if (tid == 0) counter_reset(&g_cnt_gu[a * nbn + nb]);
    if (tid < 256) S.tot[tid] = sum_agent(A.part_gu + (size_t)(a * nbn + nb) * ksn * 256 + tid, ksn, 256);
    __syncthreads();
    if (wv != 0) return;
    float g0 = S.tot[2 * l], g1 = S.tot[2 * l + 1], u0 = S.tot[128 + 2 * l], u1 = S.tot[129 + 2 * l];
    wave_fwht128(g0, g1);
    wave_fwht128(u0, u1);
    const int c = nb * 128 + 2 * l;
    g0 = (float)(half_t)(g0 * kRsqrt128 * (float)sc_g.x);
    g1 = (float)(half_t)(g1 * kRsqrt128 * (float)sc_g.y);
    u0 = (float)(half_t)(u0 * kRsqrt128 * (float)sc_u.x);
    u1 = (float)(half_t)(u1 * kRsqrt128 * (float)sc_u.y);
    float a0 = (float)(half_t)(g0 / (1.0f + expf(-g0)) * u0);
    float a1 = (float)(half_t)(g1 / (1.0f + expf(-g1)) * u1);
    a0 = (float)(half_t)(a0 * (float)sc_d.x);
    a1 = (float)(half_t)(a1 * (float)sc_d.y);
    wave_fwht128(a0, a1);
    const half2_t hv = half2_t{(half_t)(a0 * kRsqrt128), (half_t)(a1 * kRsqrt128)};
    __hip_atomic_store((uint32_t*)(A.abuf + (size_t)a * I + c), __builtin_bit_cast(uint32_t, hv), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    wait_stores();
    if (l == 0) counter_add(&g_ready[a], 1);
}

// down WG per (pair, 128-column block of H) over the full K = I: the 4-row chunks of the I/16 tile-rows go round-robin
// to the eight waves, the per-wave column sums are reduced in LDS in wave order (no cross-WG exchange), then the output
// Hadamard * w * svh_d -> y, and the combine.
template <int K>
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
    const int nch = (kt / 4 + kWaves - 1 - wv) / kWaves;      // 4-row chunks of this wave: q = wv + kWaves * c
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
    if (tid == 0) {                              // wait for the pair's whole abuf (all I/128 gate/up epilogues)
        int64_t f = !A.fused && A.fill ? A.fill[e] : 0;
        if (A.fused && miss) {                   // the write-through target is the ensure's decision
            wait_count(&g_cnt_all[2], 1);
            f = ld_agent_i64(A.fill + e);
        }
        if (f && A.n_vict_wg) wait_count(&g_cnt_all[1], A.n_vict_wg);      // and for the victims' old bytes
        S.fdst = f;
        int it = 0;
        while (__hip_atomic_load(&g_ready[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < I / 128) {
            __builtin_amdgcn_s_sleep(1);
            if (++it > kSpinMax) {
                atomicAdd(&g_status[0], 1);
                break;
            }
        }
    }
    __syncthreads();
    uint32_t* trd = S.fdst ? (uint32_t*)((uint8_t*)S.fdst + A.g.gu_bytes) : nullptr;
    half2_t* xs = S.xd;                          // abuf of the pair, [I/2] half2
    for (int i = tid; i < I / 2; i += kThreads)
        xs[i] = __builtin_bit_cast(half2_t, __hip_atomic_load((const uint32_t*)(A.abuf + (size_t)a * I) + i,
                                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    __syncthreads();
    float acc[GV::NCP][2], tacc[GV::NCP][2];
    float xsum = 0.f;
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) acc[cp][0] = acc[cp][1] = 0.f;
    for (int c = 0; c < nch; ++c) {
        const int r0 = (wv + kWaves * c) * 4;
        GV& gc = (c & 1) ? g1 : g0;
        if (trd) gc.write_through(trd, tiles_n, r0, ct0);
        gc.compute(0, xs + r0 * 8, tacc);
        if (c + 2 < nch) gc.load(tr, tiles_n, r0 + 8 * kWaves, ct0);
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
    if (wv != 0) return;
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        v0 += S.red[w][2 * l];
        v1 += S.red[w][2 * l + 1];
    }
    wave_fwht128(v0, v1);
    const int c = nb * 128 + 2 * l;
    const float sc = kRsqrt128 * wgt;
    float* y = A.ybuf + (size_t)a * H + c;
    st_agent(y, v0 * sc * (float)sc_d.x);
    st_agent(y + 1, v1 * sc * (float)sc_d.y);
    // combine: the last pair of row m to finish this 128-column block sums the top-k outputs in k order
    wait_stores();
    int old = 0;
    if (l == 0) old = counter_add(&g_cnt_c[m * nbn + nb], 1);
    old = __shfl(old, 0, 64);
    if (old != A.topk - 1) return;
    if (l == 0) counter_reset(&g_cnt_c[m * nbn + nb]);
    const float* yb = A.ybuf + (size_t)(m * A.topk) * H + c;
    float o0 = 0.f, o1 = 0.f;
    for (int k0 = 0; k0 < A.topk; k0 += 16) {    // one round of loads for up to 16 picks
        float v[16][2];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool ok = k0 + j < A.topk;
            v[j][0] = ok ? ld_agent(yb + (size_t)(k0 + j) * H) : 0.f;
            v[j][1] = ok ? ld_agent(yb + (size_t)(k0 + j) * H + 1) : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (k0 + j < A.topk) {
                o0 += v[j][0];
                o1 += v[j][1];
            }
    }
    const size_t oo = (size_t)m * A.out_stride + c;
    st_act(A.out, A.x_dt, oo, o0);
    st_act(A.out, A.x_dt, oo + 1, o1);
    // the last (row, block) of the layer: clear the ready counts and commit the cache fills
    if (l == 0) old = counter_add(&g_cnt_all[0], 1);
    old = __shfl(old, 0, 64);
    if (old != A.M * nbn - 1) return;
    if (l == 0) {
        counter_reset(&g_cnt_all[0]);
        if (A.n_vict_wg) {                       // every victim workgroup has counted itself: clear for the next call
            wait_count(&g_cnt_all[1], A.n_vict_wg);
            counter_reset(&g_cnt_all[1]);
        }
        if (A.fused) wait_count(&g_cnt_all[2], 1);
    }
    for (int i = l; i < A.npairs; i += 64) counter_reset(&g_ready[i]);
    if (A.fused) {
        // the ensure's in-place rewrite of the caller's picks (masked -> safe expert, weight 0), deferred to here
        // because every pair read them during the call; the mask rule gives the same answer now (see pair_lookup)
        const EnsureArgs& Q = A.ens;
        if (Q.ram_res) {
            const int kb = Q.layer * A.E, safe = Q.safe[Q.layer];
            for (int i = l; i < A.npairs; i += 64) {
                const int id = min(max(Q.ids[i], 0), A.E - 1);
                if (!Q.ram_res[kb + id] && Q.slot_of[kb + id] < 0) {
                    Q.ids[i] = safe;
                    Q.w[i] = 0.f;
                }
            }
        }
        const int nf = A.commit_ptrs ? ld_agent_i32(A.fill_list) : 0;
        for (int i = l; i < nf; i += 64) {
            const int ef = ld_agent_i32(A.fill_list + 1 + i);
            A.commit_ptrs[ef] = ld_agent_i64(A.commit_fill + ef);
            A.commit_fill[ef] = 0;
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

template <int K>
__global__ void __launch_bounds__(kThreads) moe_layer_kernel(DecodeArgs A) {
    __shared__ __align__(16) uint8_t lds[sizeof(LayerShared) > sizeof(EnsureShared) ? sizeof(LayerShared)
                                                                                     : sizeof(EnsureShared)];
    LayerShared& S = *reinterpret_cast<LayerShared*>(lds);
    const int nv = A.n_vict_wg;
    const int n_gu = A.npairs * (A.g.I / 128) * gu_slices(A.g.H);
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
    else down_wg<K>(A, b - nv - n_gu, S);
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

hipError_t launch_moe_layer(int K, const DecodeArgs& a, hipStream_t s) {
    const int n_gu = a.npairs * (a.g.I / 128) * gu_slices(a.g.H);
    const int n_dn = a.npairs * (a.g.H / 128);
    dim3 grid((unsigned)(a.fused + a.n_vict_wg + n_gu + n_dn));
    if (K == 2) hipLaunchKernelGGL(moe_layer_kernel<2>, grid, dim3(kThreads), 0, s, a);
    else if (K == 3) hipLaunchKernelGGL(moe_layer_kernel<3>, grid, dim3(kThreads), 0, s, a);
    else if (K == 4) hipLaunchKernelGGL(moe_layer_kernel<4>, grid, dim3(kThreads), 0, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

int read_status(int* out, hipStream_t s) {
    return (int)hipMemcpyFromSymbolAsync(out, HIP_SYMBOL(g_status), sizeof(int) * 4, 0, hipMemcpyDeviceToHost, s);
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
