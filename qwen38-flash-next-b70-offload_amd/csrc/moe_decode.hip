// Decode-size routed-expert MoE (pair mode: one row per (token, expert) pair), EXL3 trellis dequantization fused into
// the expert GEMVs, for CDNA4.
//
//   gateup_kernel : WG per (pair, 128-column block of I, 128-row block of H). Fused input Hadamard of x*suh for gate
//                   and up, trellis GEMV (one period per lane, bfe + mul + sad + fma_mix per weight), split-K partials;
//                   the last-arriving WG of a (pair, block) reduces the partials in fixed order and runs the epilogue
//                   (output Hadamards * svh, SiLU(g)*u, *suh_d, down-input Hadamard) -> abuf (fp16).
//   down_kernel   : WG per (pair, 128-column block of H, 128-row block of I): GEMV of abuf against the down trellis,
//                   last-arriver epilogue (output Hadamard * w * svh_d) -> y (fp32); the last pair of a (row, block)
//                   sums the top-k y's in k order into out (the combine), and the last (row, block) commits the
//                   expert-cache fills (ptrs[e] = fill[e]; fill[e] = 0).
//   dequant_kernel: bit-exact fp16 W_inner of one trellis matrix.
//
// Reference semantics: kernels/moe-a8/exl3_moe.a8.sycl GateUpKernel (121-260), DownKernel (264-368), CombineKernel
// (371-395); kernels/moe-a8/exl3_esimd.h ReconstructKernel (869-936). Accumulation is fp32 throughout (the reference
// keeps fp16 partials per tile-row); the fp16 rounding points of the epilogues are the reference's.
//
// The codebook affine w = c1*h + c2 is applied to the dot product: sum_k w_k x_k = c1 sum_k h_k x_k + c2 sum_k x_k,
// with h the exact fp16 1024 + bytesum, so the inner loop is bfe, mul, sad and one mixed-precision FMA per weight.
#include "exl3_common.cuh"
#include "exl3_geom.h"
#include "exl3_kernels.h"

namespace exl3 {

__device__ int g_cnt_gu[kMaxPairs * 64];
__device__ int g_cnt_d[kMaxPairs * 64];
__device__ int g_cnt_c[kMaxRows * 64];
__device__ int g_cnt_all[4];

// word offset of (tile-row r, tile-col `tile`, period p, plane i) in a PLANAR4 matrix with tiles_n tile-columns
template <int K>
__device__ __forceinline__ size_t word_off(int r, int tiles_n, int tile, int p, int i) {
    using GM = Geo<K>;
    if constexpr (GM::D > 1) {
        return (size_t)r * tiles_n * GM::W + (size_t)(tile >> 2) * 4 * GM::W + i * 4 * GM::G + (tile & 3) * GM::G + p;
    } else {
        return (size_t)r * tiles_n * GM::W + (size_t)tile * GM::W + p;
    }
}

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

// GEMV over `nrows` (compile-time 4) tile-rows of 8 tile-columns (one 128-column block): per lane accumulators for its
// column pair, for every column pass. Optional write-through of the words it reads.
template <int K>
struct Gemv8 {
    using GM = Geo<K>;
    static constexpr int G = GM::G, D = GM::D, V = GM::V, NTW = GM::NTW, NCP = 8 / NTW, L = 32 / V;
    static constexpr int NQ = V / 8;
    static_assert(NQ >= 1, "one value octet per period at least");

    // xh: 16 half2 per tile-row... laid out [tile-row][8] half2 (128-row block = 8 tile-rows)
    __device__ __forceinline__ static void run(const uint32_t* tr, uint32_t* trd, int tiles_n, int r0, int xrow0,
                                               int col_tile0, const half2_t* xh, float (&acc)[NCP][2]) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
        const int qb = ((V * p) >> 3) & 3;
#pragma unroll
        for (int cp = 0; cp < NCP; ++cp) {
            acc[cp][0] = 0.f;
            acc[cp][1] = 0.f;
            const int tile = col_tile0 + cp * NTW + j;
            uint32_t wd[4][D];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int i = 0; i < D; ++i) wd[rr][i] = __builtin_nontemporal_load(tr + word_off<K>(r0 + rr, tiles_n, tile, p, i));
            if (trd) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                    for (int i = 0; i < D; ++i) trd[word_off<K>(r0 + rr, tiles_n, tile, p, i)] = wd[rr][i];
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint32_t prev = (uint32_t)__shfl((int)wd[rr][D - 1], src_lane, 64);
                Period<K> P;
                P.set(wd[rr], prev);
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

template <int K>
__global__ void __launch_bounds__(256) gateup_kernel(DecodeArgs A) {
    using GV = Gemv8<K>;
    const int H = A.g.H, I = A.g.I;
    const int nbn = I / 128, ksn = H / 128;
    int blk = blockIdx.x;
    const int ks = blk % ksn;
    blk /= ksn;
    const int nb = blk % nbn, a = blk / nbn;
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    const int e = min(max(A.ids[a], 0), A.E - 1);      // out-of-range ids are clamped, never dereferenced
    const int m = a / A.topk;
    const uint8_t* base = (const uint8_t*)A.ptrs[e];
    uint8_t* dst = A.fill ? (uint8_t*)A.fill[e] : nullptr;

    __shared__ half2_t xh_s[2][64];
    __shared__ float ssum[2];
    __shared__ float red[2][128];
    __shared__ int last;

    if (dst && nb == 0 && ks == 0) {            // write-through of the vector tail (suh/svh)
        const uint32_t* s = (const uint32_t*)(base + A.g.off_suh_g);
        uint32_t* d = (uint32_t*)(dst + A.g.off_suh_g);
        const int n = (int)((A.g.blob - A.g.off_suh_g) >> 2);
        for (int i = tid; i < n; i += 256) d[i] = s[i];
    }
    if (wv < 2) {                                // input Hadamard of x * suh for this 128-row block
        const half_t* suh = (const half_t*)(base + (wv ? A.g.off_suh_u : A.g.off_suh_g));
        const int k0 = ks * 128 + 2 * l;
        const size_t xo = (size_t)m * A.x_stride + k0;
        float v0 = (float)(half_t)(ld_act(A.x, A.x_dt, xo) * (float)suh[k0]);
        float v1 = (float)(half_t)(ld_act(A.x, A.x_dt, xo + 1) * (float)suh[k0 + 1]);
        wave_fwht128(v0, v1);
        const half_t h0 = (half_t)(v0 * kRsqrt128), h1 = (half_t)(v1 * kRsqrt128);
        xh_s[wv][l] = half2_t{h0, h1};
        const float s = wave_sum((float)h0 + (float)h1);
        if (l == 0) ssum[wv] = s;
    }
    __syncthreads();

    const int proj = wv & 1, hf = wv >> 1;
    float acc[GV::NCP][2];
    const uint32_t* tr = (const uint32_t*)base;
    uint32_t* trd = dst ? (uint32_t*)dst : nullptr;
    GV::run(tr, trd, 2 * I / 16, ks * 8 + hf * 4, hf * 4, proj * (I / 16) + nb * 8, xh_s[proj], acc);
    int col[GV::NCP];
    bool own[GV::NCP];
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) {
        own[cp] = GV::reduce(acc[cp], cp, col[cp]);
        if (hf == 1 && own[cp]) {
            red[proj][col[cp]] = acc[cp][0];
            red[proj][col[cp] + 8] = acc[cp][1];
        }
    }
    __syncthreads();
    if (hf == 0) {
        float* part = A.part_gu + ((size_t)(a * nbn + nb) * ksn + ks) * 256 + proj * 128;
#pragma unroll
        for (int cp = 0; cp < GV::NCP; ++cp) {
            if (own[cp]) {
                const int c0 = col[cp];
                part[c0] = kC1 * (acc[cp][0] + red[proj][c0]) + kC2 * ssum[proj];
                part[c0 + 8] = kC1 * (acc[cp][1] + red[proj][c0 + 8]) + kC2 * ssum[proj];
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(&g_cnt_gu[a * nbn + nb], 1) == ksn - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    if (wv != 0) return;
    if (l == 0) g_cnt_gu[a * nbn + nb] = 0;
    const float* pp = A.part_gu + (size_t)(a * nbn + nb) * ksn * 256;
    float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
    for (int s = 0; s < ksn; ++s) {
        const float* q = pp + s * 256;
        g0 += __builtin_nontemporal_load(q + 2 * l);
        g1 += __builtin_nontemporal_load(q + 2 * l + 1);
        u0 += __builtin_nontemporal_load(q + 128 + 2 * l);
        u1 += __builtin_nontemporal_load(q + 129 + 2 * l);
    }
    wave_fwht128(g0, g1);
    wave_fwht128(u0, u1);
    const int c = nb * 128 + 2 * l;
    const half_t* svg = (const half_t*)(base + A.g.off_svh_g) + c;
    const half_t* svu = (const half_t*)(base + A.g.off_svh_u) + c;
    const half_t* sud = (const half_t*)(base + A.g.off_suh_d) + c;
    g0 = (float)(half_t)(g0 * kRsqrt128 * (float)svg[0]);
    g1 = (float)(half_t)(g1 * kRsqrt128 * (float)svg[1]);
    u0 = (float)(half_t)(u0 * kRsqrt128 * (float)svu[0]);
    u1 = (float)(half_t)(u1 * kRsqrt128 * (float)svu[1]);
    float a0 = (float)(half_t)(g0 / (1.0f + expf(-g0)) * u0);
    float a1 = (float)(half_t)(g1 / (1.0f + expf(-g1)) * u1);
    a0 = (float)(half_t)(a0 * (float)sud[0]);
    a1 = (float)(half_t)(a1 * (float)sud[1]);
    wave_fwht128(a0, a1);
    *(half2_t*)(A.abuf + (size_t)a * I + c) = half2_t{(half_t)(a0 * kRsqrt128), (half_t)(a1 * kRsqrt128)};
}

template <int K>
__global__ void __launch_bounds__(128) down_kernel(DecodeArgs A) {
    using GV = Gemv8<K>;
    const int H = A.g.H, I = A.g.I;
    const int nbn = H / 128, ksn = I / 128;
    int blk = blockIdx.x;
    const int ks = blk % ksn;
    blk /= ksn;
    const int nb = blk % nbn, a = blk / nbn;
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
    const int e = min(max(A.ids[a], 0), A.E - 1);      // out-of-range ids are clamped, never dereferenced
    const int m = a / A.topk;
    const uint8_t* base = (const uint8_t*)A.ptrs[e];
    uint8_t* dst = A.fill ? (uint8_t*)A.fill[e] : nullptr;

    __shared__ half2_t xh_s[64];
    __shared__ float ssum;
    __shared__ float red[128];
    __shared__ int last;

    if (wv == 0) {
        const half2_t v = *(const half2_t*)(A.abuf + (size_t)a * I + ks * 128 + 2 * l);
        xh_s[l] = v;
        const float s = wave_sum((float)v.x + (float)v.y);
        if (l == 0) ssum = s;
    }
    __syncthreads();
    float acc[GV::NCP][2];
    const uint32_t* tr = (const uint32_t*)(base + A.g.gu_bytes);
    uint32_t* trd = dst ? (uint32_t*)(dst + A.g.gu_bytes) : nullptr;
    GV::run(tr, trd, H / 16, ks * 8 + wv * 4, wv * 4, nb * 8, xh_s, acc);
    int col[GV::NCP];
    bool own[GV::NCP];
#pragma unroll
    for (int cp = 0; cp < GV::NCP; ++cp) {
        own[cp] = GV::reduce(acc[cp], cp, col[cp]);
        if (wv == 1 && own[cp]) {
            red[col[cp]] = acc[cp][0];
            red[col[cp] + 8] = acc[cp][1];
        }
    }
    __syncthreads();
    if (wv == 0) {
        float* part = A.part_d + ((size_t)(a * nbn + nb) * ksn + ks) * 128;
#pragma unroll
        for (int cp = 0; cp < GV::NCP; ++cp) {
            if (own[cp]) {
                const int c0 = col[cp];
                part[c0] = kC1 * (acc[cp][0] + red[c0]) + kC2 * ssum;
                part[c0 + 8] = kC1 * (acc[cp][1] + red[c0 + 8]) + kC2 * ssum;
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(&g_cnt_d[a * nbn + nb], 1) == ksn - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    if (wv != 0) return;
    if (l == 0) g_cnt_d[a * nbn + nb] = 0;
    const float* pp = A.part_d + (size_t)(a * nbn + nb) * ksn * 128;
    float v0 = 0.f, v1 = 0.f;
    for (int s = 0; s < ksn; ++s) {
        v0 += __builtin_nontemporal_load(pp + s * 128 + 2 * l);
        v1 += __builtin_nontemporal_load(pp + s * 128 + 2 * l + 1);
    }
    wave_fwht128(v0, v1);
    const int c = nb * 128 + 2 * l;
    const half_t* svd = (const half_t*)(base + A.g.off_svh_d) + c;
    const float sc = kRsqrt128 * A.w[a];
    float* y = A.ybuf + (size_t)a * H + c;
    y[0] = v0 * sc * (float)svd[0];
    y[1] = v1 * sc * (float)svd[1];
    // combine: the last pair of row m to finish this 128-column block sums the top-k outputs in k order
    __threadfence();
    int old = 0;
    if (l == 0) old = atomicAdd(&g_cnt_c[m * nbn + nb], 1);
    old = __shfl(old, 0, 64);
    if (old != A.topk - 1) return;
    __threadfence();
    if (l == 0) g_cnt_c[m * nbn + nb] = 0;
    float o0 = 0.f, o1 = 0.f;
    for (int k = 0; k < A.topk; ++k) {
        const float* yk = A.ybuf + (size_t)(m * A.topk + k) * H + c;
        o0 += __builtin_nontemporal_load(yk);
        o1 += __builtin_nontemporal_load(yk + 1);
    }
    const size_t oo = (size_t)m * A.out_stride + c;
    st_act(A.out, A.x_dt, oo, o0);
    st_act(A.out, A.x_dt, oo + 1, o1);
    if (!A.commit_ptrs) return;
    __threadfence();
    if (l == 0) old = atomicAdd(&g_cnt_all[0], 1);
    old = __shfl(old, 0, 64);
    if (old != A.M * nbn - 1) return;
    __threadfence();
    if (l == 0) g_cnt_all[0] = 0;
    const int nf = A.fill_list[0];
    for (int i = l; i < nf; i += 64) {
        const int ef = A.fill_list[1 + i];
        A.commit_ptrs[ef] = A.commit_fill[ef];
        A.commit_fill[ef] = 0;
    }
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

hipError_t launch_gateup(int K, const DecodeArgs& a, hipStream_t s) {
    dim3 grid((unsigned)(a.npairs * (a.g.I / 128) * (a.g.H / 128)));
    if (K == 2) hipLaunchKernelGGL(gateup_kernel<2>, grid, dim3(256), 0, s, a);
    else if (K == 3) hipLaunchKernelGGL(gateup_kernel<3>, grid, dim3(256), 0, s, a);
    else if (K == 4) hipLaunchKernelGGL(gateup_kernel<4>, grid, dim3(256), 0, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_down(int K, const DecodeArgs& a, hipStream_t s) {
    dim3 grid((unsigned)(a.npairs * (a.g.H / 128) * (a.g.I / 128)));
    if (K == 2) hipLaunchKernelGGL(down_kernel<2>, grid, dim3(128), 0, s, a);
    else if (K == 3) hipLaunchKernelGGL(down_kernel<3>, grid, dim3(128), 0, s, a);
    else if (K == 4) hipLaunchKernelGGL(down_kernel<4>, grid, dim3(128), 0, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
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
