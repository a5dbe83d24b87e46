// The dense EXL3 linear on gfx950: out[M, n] = svh * H(sum_k xh[g(n)][m][k] W[k][n]) / sqrt 128, with
// xh[g] = fp16(H(fp16(x * suh[g])) / sqrt 128) per shard g and W the codebook values of a trellis in the checkpoint's
// natural word order (reference: experimental/n111-victim-ring/csrc/exl3_ops.sycl:651-757; HadInKernel /
// HadOutKernel, exl3_esimd.h:286-343; ReconstructKernel, exl3_esimd.h:869-936). Codebooks: mul1 at K = 2..6, and
// 3inst / mcg at K = 4 and 6 (the reference's EXL3_ALL_CODEBOOKS set, exl3_ops.sycl:767-773).
//
// Small M (<= kLinMaxRows), one launch: a workgroup of 4 waves takes 4 consecutive 128-row blocks (one K-slice) of
// one 64-column group; each wave computes the input Hadamards of its own block for every row in registers, then runs
// the 8 x 4-tile dequant-GEMV (the MoE gate/up wave GEMV on natural-order words), every codebook value decoded once
// and multiplied into all M rows (mul1: on the raw codebook integers, sum w x = c1 sum h x + c2 sum x; 3inst / mcg:
// on the fp16 weights themselves). The 4 waves are
// summed in LDS into one fp32 partial per K-slice. The 2P workgroups of a 128-column block hand their partials to the
// block's last workgroup in dispatch order as tagged 64-bit words ((1 << 32) | fp32 bits, agent scope); it polls them
// (all loads of a round in flight together; bounded, a timeout counted in the device status words), sums the P slices
// in order, applies the output Hadamard x svh and clears the words it read, so the exchange area is zero between
// calls and needs no counter or epoch. k <= 512 (one slice): one workgroup of 8 waves per 128-column block, no hand-off.
// Large M: the input-Hadamard kernel, fp16 W slices (lin_reconstruct_kernel) for a library GEMM, then the output
// kernel on its fp16 product.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "exl3_common.cuh"
#include "exl3_gemv.cuh"
#include "exl3_kernels.h"

namespace exl3 {

constexpr int kLinWaves = 4;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// The 8 x 4-tile wave GEMV with the multiply-adds on the matrix cores (v_mfma_f32_16x16x32_f16, the full-rate shape
// on gfx950), for the bitrates whose trellis period is 2 columns x 16 rows of a tile (V = 32: K = 3, 5). A pass covers
// 4 tile-rows x 2 tile-columns: lane l decodes period l & 7 of tile-row 4 (ps & 1) + (l >> 4), tile-column
// 2 (ps >> 1) + ((l >> 3) & 1), so the 16 lanes of MFMA k-group q = l >> 4 share one tile-row and each lane's period
// holds the 8-row halves (rows 8 i .. 8 i + 7) of its two columns p and p + 8 that the B operand needs. The B values are the raw codebook integers h (exact in fp16,
// two packed per register); A = the rows' xh over the same 4-row slices (zero for rows past MR); the raw-h affine is
// applied to the column sums as in the VALU version. VALU per weight: bfe, mul and sad (v_sad_hi_u8 packs the pair),
// for any MR.
template <int K>
struct GemvMfma {
    static constexpr int D = Geo<K>::D;
    static_assert(Geo<K>::V == 32 && Geo<K>::G == 8, "the MFMA layout needs periods of 2 columns x 16 rows");
    uint32_t wd[4][D];

    __device__ __forceinline__ void load_nat(const uint32_t* tr, int tiles_n, int rt0, int ct0) {
        const int l = lane_id(), q = l >> 4, c = (l >> 3) & 1, p = l & 7;
#pragma unroll
        for (int ps = 0; ps < 4; ++ps)
#pragma unroll
            for (int i = 0; i < D; ++i)
                wd[ps][i] = __builtin_nontemporal_load(
                    as_global(tr) + word_off_nat<K>(rt0 + 4 * (ps & 1) + q, tiles_n, ct0 + 2 * (ps >> 1) + c, p, i));
    }

    // raw h of values u and u + 1 packed into one register (h of u in the low half)
    template <int u>
    __device__ __forceinline__ static uint32_t pair(const Period<K>& P) {
        return cb_raw2(P.template state<u>(), P.template state<u + 1>());
    }
    // rows 8 i .. 8 i + 7 of column p + 8 h: u = 2 i + 4 h + {0, 1, 8, 9, 16, 17, 24, 25} in row order
    template <int i, int h>
    __device__ __forceinline__ static half8_t bop(const Period<K>& P) {
        constexpr int u0 = 2 * i + 4 * h;
        typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(half8_t, u4_t{pair<u0>(P), pair<u0 + 8>(P), pair<u0 + 16>(P), pair<u0 + 24>(P)});
    }
    template <int MR, int i>
    __device__ __forceinline__ static void step(const Period<K>& P, const half2_t* xq, int xrow, float4_t (&acc)[2]) {
        const int m = lane_id() & 15;
        half8_t a = half8_t{};
        if (m < MR) a = *(const half8_t*)(xq + m * 64 + (xrow + 8 * i) / 2);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop<i, 0>(P), acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop<i, 1>(P), acc[1], 0, 0, 0);
    }

    // xq = [MR][64] half2 (the wave's 128-row block of each row); acc[pair of tile-columns][h]: D[m][n] with lane l
    // holding rows m = 4 (l >> 4) .. + 3 of column n = l & 15 (tile-column (n >> 3) & 1 of the pair, column n & 7 + 8 h)
    template <int MR>
    __device__ __forceinline__ void compute(const half2_t* xq, float4_t (&acc)[2][2]) const {
        const int l = lane_id(), q = l >> 4;
        const int src = (l & ~7) | ((l + 7) & 7);
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
            const uint32_t prev = (uint32_t)__shfl((int)wd[ps][D - 1], src, 64);
            Period<K> P;
            P.set(wd[ps], prev);
            const int xrow = 16 * (4 * (ps & 1) + q);
            step<MR, 0>(P, xq, xrow, acc[ps >> 1]);
            step<MR, 1>(P, xq, xrow, acc[ps >> 1]);
        }
    }
};
// MFMA from 4 rows on (at 1 and 2 rows the VALU multiply-adds cost less than the MFMA path's operand handling:
// 7.7 / 8.8 us against 8.2 / 8.9 us per call at bs 1 / 2 on the 48-layer dense workload; 10.2 / 13.5 against
// 10.8 / 15.8 at bs 4 / 8)
template <int K, int MR, int CB = 2> constexpr bool kLinMfma = CB == 2 && Geo<K>::V == 32 && Geo<K>::G == 8 && MR >= 4;
template <int K, bool M> struct LinGemvSel { using type = Gemv4<K>; };
template <int K> struct LinGemvSel<K, true> { using type = GemvMfma<K>; };

// one wave per (shard g, row m, 128-block kb)
__global__ void __launch_bounds__(256) lin_had_in_kernel(LinearArgs A) {
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), l = lane_id();
    const int kbn = A.k / 128;
    if (wave >= A.S * A.M * kbn) return;
    const int kb = wave % kbn, m = (wave / kbn) % A.M, g = wave / (kbn * A.M);
    const size_t xo = (size_t)m * A.x_stride + kb * 128 + 2 * l;
    const half_t* su = A.suh + (size_t)g * A.k + kb * 128 + 2 * l;
    float v0 = (float)to_half(ld_act(A.x, A.x_dt, xo) * (float)su[0]);
    float v1 = (float)to_half(ld_act(A.x, A.x_dt, xo + 1) * (float)su[1]);
    wave_fwht128(v0, v1);
    *(half2_t*)(A.xh + ((size_t)g * A.M + m) * A.k + kb * 128 + 2 * l) =
        half2_t{to_half(v0 * kRsqrt128), to_half(v1 * kRsqrt128)};
}

// tagged hand-off words of the small-M path: (1 << 32) | fp32 bits; zero (cleared) between calls
__device__ __forceinline__ void lin_st_tag(uint64_t* p, float v) {
    __hip_atomic_store(p, (1ull << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t lin_ld(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lin_clear(uint64_t* p) {
    __hip_atomic_store(p, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kLinSpinMax = 1 << 22;
// bounded poll bookkeeping: true once the budget is spent (counted in the device status words and their host mirror)
__device__ __forceinline__ bool lin_spin_out(const LinearArgs& A, int& it) {
    if (++it > kLinSpinMax) {
        if (lane_id() == 0 && A.status) {
            atomicAdd(A.status, 1);
            int* h = *A.status_host;
            if (h) __hip_atomic_fetch_add(h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        return true;
    }
    __builtin_amdgcn_s_sleep(1);
    return false;
}

// One wave's share: the weights of 128-row block kb x 64-column group cg (loads issued first), the input Hadamards of
// that block for every row into xqw [MR][64] (their sums into sswv [MR]), the dequant-GEMV, and the wave's 64 column
// sums per row into redw [MR][64]
template <int K, int MR, int CB>
__device__ __forceinline__ void lin_wave(const LinearArgs& A, int kb, int cg, int nb, half2_t (*xqw)[64], float* sswv,
                                         float (*redw)[64]) {
    using GQ = typename LinGemvSel<K, kLinMfma<K, MR, CB>>::type;
    const int kbn = A.k / 128, l = lane_id();
    const bool in_k = kb < kbn;                  // waves past the end of k add nothing
    // the loads that depend on nothing go first: the activations (raw bits), every shard's suh row of the block (up
    // to 4 shards, beside the shard index, so that no load waits for another), then the weights; the Hadamard waits
    // only for the first two
    uint64_t xr[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        xr[m] = 0;
        if (in_k && m < A.M) {
            const size_t xo = (size_t)m * A.x_stride + kb * 128 + 2 * l;
            xr[m] = ld_act2_raw(A.x, A.x_dt, xo);
        }
    }
    const int g = A.shard_of_nb[nb];
    const size_t so = (size_t)min(kb, kbn - 1) * 128 + 2 * l;
    uint32_t sus[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sus[j] = *(const uint32_t*)(A.suh + (size_t)min(j, A.S - 1) * A.k + so);
    GQ gv;
    if (in_k) gv.load_nat(A.tr, A.n / 16, kb * 8, cg * 4);
    float xv[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) act2_cvt(xr[m], A.x_dt, xv[m][0], xv[m][1]);
    const bool live = in_k && (unsigned)g < (unsigned)A.S;   // a shard index outside [0, S) leaves its columns zero
    uint32_t suw = 0;
    if (live) suw = A.S > 4 ? *(const uint32_t*)(A.suh + (size_t)g * A.k + so)
                            : g == 0 ? sus[0] : g == 1 ? sus[1] : g == 2 ? sus[2] : sus[3];
    const half2_t su = __builtin_bit_cast(half2_t, suw);
#pragma unroll
    for (int m = 0; m < MR; ++m) {               // xh = fp16(H(fp16(x su)) / sqrt 128) of this block, and its sum
        float v0 = 0.f, v1 = 0.f;
        if (live && m < A.M) {
            v0 = (float)to_half(xv[m][0] * (float)su.x);
            v1 = (float)to_half(xv[m][1] * (float)su.y);
        }
        wave_fwht128(v0, v1);
        const half2_t v = half2_t{to_half(v0 * kRsqrt128), to_half(v1 * kRsqrt128)};
        xqw[m][l] = v;
        const float s = wave_sum((float)v.x + (float)v.y);
        if (l == 0) sswv[m] = s;
    }
    if constexpr (kLinMfma<K, MR, CB>) {
        float4_t acc[2][2];
#pragma unroll
        for (int c = 0; c < 2; ++c)
            acc[c][0] = acc[c][1] = float4_t{0.f, 0.f, 0.f, 0.f};
        if (live) gv.template compute<MR>(&xqw[0][0], acc);      // the wave's own LDS rows: no barrier
        const int n = l & 15, q4 = 4 * (l >> 4);
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (q4 + v < MR) redw[q4 + v][16 * (2 * c + ((n >> 3) & 1)) + 8 * h + (n & 7)] = acc[c][h][v];
    } else {
        float acc[MR][GQ::NCQ][2];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int q = 0; q < GQ::NCQ; ++q) acc[m][q][0] = acc[m][q][1] = 0.f;
        if (live) gv.template compute_mr<MR, CB>(&xqw[0][0], acc);     // the wave's own LDS rows: no barrier
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int q = 0; q < GQ::NCQ; ++q) {
                int c0;
                if (GQ::reduce(acc[m][q], q, c0)) {
                    redw[m][c0] = acc[m][q][0];
                    redw[m][c0 + 8] = acc[m][q][1];
                }
            }
    }
}

// a K-slice's column sum from its 4 blocks' raw sums t and activation sums xs: mul1 applies the codebook affine here
template <int CB>
__device__ __forceinline__ float lin_colsum(float t, float xs) {
    if constexpr (CB == 2) return kC1 * t + kC2 * xs;
    else return t;
}

template <int K, int MR, int CB>
__global__ void __launch_bounds__(64 * kLinWaves) lin_small_kernel(LinearArgs A, void* out, int out_dt,
                                                                  int64_t out_stride) {
    constexpr int RPW = (MR + kLinWaves - 1) / kLinWaves;   // output rows per wave of the owner
    __shared__ half2_t xq[kLinWaves][MR][64];
    __shared__ float ssw[kLinWaves][MR];
    __shared__ float red[kLinWaves][MR][64];
    __shared__ float own[MR][64];
    const int P = A.P;
    const int cg = blockIdx.x / P, ks = blockIdx.x % P, nb = cg >> 1;
    const int wv = threadIdx.x >> 6, l = lane_id();
    const bool owner = (cg & 1) && ks == P - 1;   // the block's last workgroup in dispatch order
    lin_wave<K, MR, CB>(A, ks * kLinWaves + wv, cg, nb, xq[wv], ssw[wv], red[wv]);
    __syncthreads();
    for (int i = threadIdx.x; i < MR * 64; i += 64 * kLinWaves) {
        const int m = i >> 6, c = i & 63;
        if (m >= A.M) continue;
        float t = 0.f, xs = 0.f;                 // the 4 blocks in order
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) {
            t += red[w][m][c];
            xs += ssw[w][m];
        }
        const float v = lin_colsum<CB>(t, xs);
        if (owner) own[m][c] = v;
        else lin_st_tag(A.part + ((size_t)ks * A.M + m) * A.n + cg * 64 + c, v);
    }
    if (!owner) return;
    __syncthreads();
    // the block's output rows m = wv + r * 4: lane l sums columns 2l, 2l + 1 of block nb over the P slices in order;
    // lanes 32.. take slice P - 1 from this workgroup's own partial. Up to 8 slices of all the wave's rows are polled
    // together (every load issued before any tag is checked).
    if (wv >= A.M) return;                       // no output row for this wave
    const half2_t sv = *(const half2_t*)(A.svh + nb * 128 + 2 * l);
    const bool hi = l >= 32;
    const size_t sstride = (size_t)A.M * A.n;
    float v0[RPW], v1[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) v0[r] = v1[r] = 0.f;
    for (int s0 = 0; s0 < P; s0 += 8) {
        const int ns = min(8, P - s0);
        uint64_t w[RPW][8][2];
        int it = 0;
        for (;;) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const int m = min(wv + r * kLinWaves, A.M - 1);
                const uint64_t* q = A.part + (size_t)m * A.n + nb * 128 + 2 * l;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const size_t o = (size_t)min(s0 + j, P - 1) * sstride;
                    w[r][j][0] = lin_ld(q + o);
                    w[r][j][1] = lin_ld(q + o + 1);
                }
            }
            bool ok = true;
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const bool need = wv + r * kLinWaves < A.M && j < ns && !(hi && s0 + j == P - 1);
                    ok &= !need | (((uint32_t)(w[r][j][0] >> 32) == 1u) & ((uint32_t)(w[r][j][1] >> 32) == 1u));
                }
            if (__all(ok) || lin_spin_out(A, it)) break;
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int m = wv + r * kLinWaves;
            if (m >= A.M) continue;
            uint64_t* q = A.part + (size_t)m * A.n + nb * 128 + 2 * l;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int sl = s0 + j;
                if (j >= ns) continue;
                if (hi && sl == P - 1) {
                    v0[r] += own[m][2 * l - 64];
                    v1[r] += own[m][2 * l - 63];
                } else {
                    v0[r] += __uint_as_float((uint32_t)w[r][j][0]);
                    v1[r] += __uint_as_float((uint32_t)w[r][j][1]);
                    lin_clear(q + sl * sstride);
                    lin_clear(q + sl * sstride + 1);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int m = wv + r * kLinWaves;
        if (m >= A.M) continue;
        float a0 = v0[r], a1 = v1[r];
        wave_fwht128(a0, a1);
        const size_t o = (size_t)m * out_stride + nb * 128 + 2 * l;
        st_act(out, out_dt, o, a0 * kRsqrt128 * (float)sv.x);
        st_act(out, out_dt, o + 1, a1 * kRsqrt128 * (float)sv.y);
    }
}

// one wave per (row m, 128-column block nb)
template <typename TPart>
__global__ void __launch_bounds__(256) lin_had_out_kernel(const TPart* part, int P, int M, int n, const half_t* svh,
                                                          void* out, int out_dt, int64_t out_stride) {
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), l = lane_id();
    const int nbn = n / 128;
    if (wave >= M * nbn) return;
    const int nb = wave % nbn, m = wave / nbn;
    float v0 = 0.f, v1 = 0.f;
    for (int p = 0; p < P; ++p) {                // the K-slices in order
        const TPart* q = part + ((size_t)p * M + m) * n + nb * 128 + 2 * l;
        v0 += (float)q[0];
        v1 += (float)q[1];
    }
    wave_fwht128(v0, v1);
    const half2_t sv = *(const half2_t*)(svh + nb * 128 + 2 * l);
    const size_t o = (size_t)m * out_stride + nb * 128 + 2 * l;
    st_act(out, out_dt, o, v0 * kRsqrt128 * (float)sv.x);
    st_act(out, out_dt, o + 1, v1 * kRsqrt128 * (float)sv.y);
}

// ---- the W8A8 route of the large-M linear (exl3_ops.sycl:520-537, 668-740; opt-in): every mul1 codebook value lies
// in [-3.453125, 3.453125], so one static int8 scale serves all weights; the activations get one scale per (shard,
// row), the GEMM runs on int8 with int32 sums ------------------------------------------------------------------------

constexpr float kQ8WMax = 3.453125f;             // the largest |mul1 codebook value| (exl3_ops.sycl:526)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, lane_xor(v, m));
    return v;
}

// xq[g][m][:] = int8(rne(xh * inv)) and sx[g][m] = sc, with xh the fp16 path's input Hadamard of row m for shard g,
// amax its largest magnitude, sc = amax / 127 (1 for an all-zero row) and inv = 1 / sc (HadInQ8Kernel and
// HadInQ8WgKernel, exl3_esimd.h:341-421). One workgroup of 8 waves per (g, m), wave w taking blocks w, w + 8, ...:
// with NB > 0 each wave keeps its (at most NB) blocks in registers between the row maximum and the quantization;
// NB = 0 (rows of more than 16,384) recomputes each block for the second pass.
constexpr int kQ8Waves = 8;
template <int NB>
__global__ void __launch_bounds__(64 * kQ8Waves) lin_had_in_q8_kernel(LinearArgs A, int8_t* __restrict__ xq,
                                                                      float* __restrict__ sx, int64_t ms) {
    __shared__ float wmax[kQ8Waves];
    const int m = blockIdx.x % A.M, g = blockIdx.x / A.M;
    const int wv = threadIdx.x >> 6, l = lane_id(), kbn = A.k / 128;
    const half_t* su = A.suh + (size_t)g * A.k + 2 * l;
    auto block = [&](int kb, float& v0, float& v1) {    // the fp16 path's xh of block kb (whole wave)
        const size_t xo = (size_t)m * A.x_stride + kb * 128 + 2 * l;
        v0 = (float)to_half(ld_act(A.x, A.x_dt, xo) * (float)su[kb * 128]);
        v1 = (float)to_half(ld_act(A.x, A.x_dt, xo + 1) * (float)su[kb * 128 + 1]);
        wave_fwht128(v0, v1);
        v0 = (float)to_half(v0 * kRsqrt128);
        v1 = (float)to_half(v1 * kRsqrt128);
    };
    constexpr int NR = NB > 0 ? NB : 1;
    float v[NR][2];
    float mx = 0.f;
    if constexpr (NB > 0) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {           // kb depends on the wave only: whole waves stay together
            const int kb = wv + kQ8Waves * j;
            v[j][0] = v[j][1] = 0.f;
            if (kb < kbn) block(kb, v[j][0], v[j][1]);
            mx = fmaxf(mx, fmaxf(fabsf(v[j][0]), fabsf(v[j][1])));
        }
    } else {
        for (int kb = wv; kb < kbn; kb += kQ8Waves) {
            block(kb, v[0][0], v[0][1]);
            mx = fmaxf(mx, fmaxf(fabsf(v[0][0]), fabsf(v[0][1])));
        }
    }
    mx = wave_max(mx);
    if (l == 0) wmax[wv] = mx;
    __syncthreads();
    float amax = wmax[0];
#pragma unroll
    for (int w = 1; w < kQ8Waves; ++w) amax = fmaxf(amax, wmax[w]);
    const float sc = amax > 0.f ? amax / 127.f : 1.f;
    const float inv = 1.f / sc;
    if (threadIdx.x == 0) sx[(size_t)g * ms + m] = sc;
    int8_t* q = xq + ((size_t)g * ms + m) * A.k + 2 * l;
    auto store = [&](int kb, float v0, float v1) {
        const int q0 = (int)__builtin_rintf(v0 * inv), q1 = (int)__builtin_rintf(v1 * inv);
        *(uint16_t*)(q + kb * 128) = (uint16_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8));
    };
    if constexpr (NB > 0) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int kb = wv + kQ8Waves * j;
            if (kb < kbn) store(kb, v[j][0], v[j][1]);
        }
    } else {
        for (int kb = wv; kb < kbn; kb += kQ8Waves) {
            block(kb, v[0][0], v[0][1]);
            store(kb, v[0][0], v[0][1]);
        }
    }
}

// int8 store of one period's mul1 values: w = int8(rne(W * 127 / 3.453125)) (ReconstructKernel with an int8 output,
// exl3_esimd.h:869-936 and exl3_ops.sycl:528-537)
template <int K, int u>
__device__ __forceinline__ void dequant_store_q8(const Period<K>& P, int p, int8_t* o, size_t n_out, float inv) {
    if constexpr (u < Geo<K>::V) {
        const half2_t w = cb_w2(P.template state<u>(), P.template state<u + 1>());
        o[(size_t)val_row<K>(p, u) * n_out + val_col<K>(p, u)] = (int8_t)(int)__builtin_rintf((float)w.x * inv);
        o[(size_t)val_row<K>(p, u + 1) * n_out + val_col<K>(p, u + 1)] = (int8_t)(int)__builtin_rintf((float)w.y * inv);
        dequant_store_q8<K, u + 2>(P, p, o, n_out, inv);
    }
}

// out[m, c] = svh[c] * H(y[m, :] * (sx[m] * sw)) / sqrt 128 over the ng columns of one shard group, y int32 [M][ng]
// (HadOutQ8Kernel, exl3_esimd.h:423-440): one wave per (row, 128-column block)
__global__ void __launch_bounds__(256) lin_had_out_q8_kernel(const int32_t* __restrict__ y, const float* __restrict__ sx,
                                                             float sw, int M, int ng, const half_t* __restrict__ svh,
                                                             void* out, int out_dt, int64_t out_stride) {
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), l = lane_id();
    const int nbn = ng / 128;
    if (wave >= M * nbn) return;                 // whole waves
    const int nb = wave % nbn, m = wave / nbn;
    const int32_t* yr = y + (size_t)m * ng + nb * 128 + 2 * l;
    const float s = sx[m] * sw;
    float v0 = (float)yr[0] * s, v1 = (float)yr[1] * s;
    wave_fwht128(v0, v1);
    const half2_t sv = *(const half2_t*)(svh + nb * 128 + 2 * l);
    const size_t o = (size_t)m * out_stride + nb * 128 + 2 * l;
    st_act(out, out_dt, o, v0 * kRsqrt128 * (float)sv.x);
    st_act(out, out_dt, o + 1, v1 * kRsqrt128 * (float)sv.y);
}

// one wave per (tile-row, strip of NTW tiles) of tile-columns [t0, t1): W[k][16 (t1 - t0)] of codebook CB, fp16
// bit-exact (TW = half_t) or, for mul1, int8 at the static scale 127 / 3.453125 (TW = int8_t)
template <int K, int CB, typename TW>
__global__ void __launch_bounds__(256) lin_reconstruct_kernel(const uint32_t* __restrict__ tr, int k_tiles,
                                                              int n_tiles, int t0, int t1, TW* __restrict__ w) {
    using GM = Geo<K>;
    constexpr int G = GM::G, D = GM::D, NTW = GM::NTW;
    const int nt = t1 - t0, strips = (nt + NTW - 1) / NTW;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= k_tiles * strips) return;
    const int r = wave / strips, st = wave % strips;
    const int l = lane_id(), p = l % G, j = l / G;
    const int tl = st * NTW + j;
    const bool ok = tl < nt;
    uint32_t wd[D];
#pragma unroll
    for (int i = 0; i < D; ++i) wd[i] = ok ? tr[word_off_nat<K>(r, n_tiles, t0 + tl, p, i)] : 0u;
    const uint32_t prev = (uint32_t)__shfl((int)wd[D - 1], j * G + ((p + G - 1) % G), 64);
    if (!ok) return;
    Period<K> P;
    P.set(wd, prev);
    const size_t ld = (size_t)nt * 16;
    if constexpr (std::is_same_v<TW, int8_t>)
        dequant_store_q8<K, 0>(P, p, w + (size_t)r * 16 * ld + (size_t)tl * 16, ld, 127.f / kQ8WMax);
    else
        dequant_store<K, 0, CB>(P, p, w + (size_t)r * 16 * ld + (size_t)tl * 16, ld);
}

// k <= 512 (one K-slice): a workgroup of 8 waves takes both 64-column groups of a 128-column block (waves 0-3 the
// first, 4-7 the second, one 128-row block each), sums the slice in LDS and applies the output Hadamard itself: no
// partials in global memory and no arrival counter. Same sums in the same order as lin_small_kernel with P = 1.
constexpr int kLin1Waves = 8;
template <int K, int MR, int CB>
__global__ void __launch_bounds__(64 * kLin1Waves) lin_small1_kernel(LinearArgs A, void* out, int out_dt,
                                                                    int64_t out_stride) {
    __shared__ half2_t xq[kLin1Waves][MR][64];
    __shared__ float ssw[kLin1Waves][MR];
    __shared__ float red[kLin1Waves][MR][64];
    __shared__ float yb[MR][128];
    const int nb = blockIdx.x;
    const int wv = threadIdx.x >> 6, l = lane_id();
    lin_wave<K, MR, CB>(A, wv & 3, 2 * nb + (wv >> 2), nb, xq[wv], ssw[wv], red[wv]);
    __syncthreads();
    for (int i = threadIdx.x; i < MR * 128; i += 64 * kLin1Waves) {
        const int m = i >> 7, c = i & 127, w0 = (c >> 6) * 4;
        if (m >= A.M) continue;
        float t = 0.f, xs = 0.f;                 // the 4 blocks in order
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            t += red[w0 + w][m][c & 63];
            xs += ssw[w][m];
        }
        yb[m][c] = 0.f + lin_colsum<CB>(t, xs);
    }
    __syncthreads();
    const half2_t sv = *(const half2_t*)(A.svh + nb * 128 + 2 * l);
    for (int m = wv; m < A.M; m += kLin1Waves) {
        float v0 = yb[m][2 * l], v1 = yb[m][2 * l + 1];
        wave_fwht128(v0, v1);
        const size_t o = (size_t)m * out_stride + nb * 128 + 2 * l;
        st_act(out, out_dt, o, v0 * kRsqrt128 * (float)sv.x);
        st_act(out, out_dt, o + 1, v1 * kRsqrt128 * (float)sv.y);
    }
}

// ---- launchers -----------------------------------------------------------------------------------------------------

hipError_t launch_linear_had_in(const LinearArgs& a, hipStream_t s) {
    const int waves = a.S * a.M * (a.k / 128);
    hipLaunchKernelGGL(lin_had_in_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int K, int MR, int CB>
static void small_launch(const LinearArgs& a, void* out, int out_dt, int64_t out_stride, hipStream_t s) {
    if (a.P == 1)
        hipLaunchKernelGGL((lin_small1_kernel<K, MR, CB>), dim3((unsigned)(a.n / 128)), dim3(64 * kLin1Waves), 0, s, a,
                           out, out_dt, out_stride);
    else
        hipLaunchKernelGGL((lin_small_kernel<K, MR, CB>), dim3((unsigned)((a.n / 64) * a.P)), dim3(64 * kLinWaves), 0,
                           s, a, out, out_dt, out_stride);
}

template <int K, int CB>
static hipError_t small_rows(const LinearArgs& a, void* out, int out_dt, int64_t out_stride, hipStream_t s) {
    if (a.M <= 1) small_launch<K, 1, CB>(a, out, out_dt, out_stride, s);
    else if (a.M <= 2) small_launch<K, 2, CB>(a, out, out_dt, out_stride, s);
    else if (a.M <= 4) small_launch<K, 4, CB>(a, out, out_dt, out_stride, s);
    else if (a.M <= kLinMaxRows) small_launch<K, kLinMaxRows, CB>(a, out, out_dt, out_stride, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// (K, codebook) pairs built: mul1 (2) at K = 2..6, 3inst (0) and mcg (1) at K = 4 and 6
hipError_t launch_linear_small(int K, int cb, const LinearArgs& a, void* out, int out_dt, int64_t out_stride,
                               hipStream_t s) {
    switch (cb * 8 + K) {
        case 16 + 2: return small_rows<2, 2>(a, out, out_dt, out_stride, s);
        case 16 + 3: return small_rows<3, 2>(a, out, out_dt, out_stride, s);
        case 16 + 4: return small_rows<4, 2>(a, out, out_dt, out_stride, s);
        case 16 + 5: return small_rows<5, 2>(a, out, out_dt, out_stride, s);
        case 16 + 6: return small_rows<6, 2>(a, out, out_dt, out_stride, s);
        case 8 + 4: return small_rows<4, 1>(a, out, out_dt, out_stride, s);
        case 8 + 6: return small_rows<6, 1>(a, out, out_dt, out_stride, s);
        case 4: return small_rows<4, 0>(a, out, out_dt, out_stride, s);
        case 6: return small_rows<6, 0>(a, out, out_dt, out_stride, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_linear_had_out(const void* parts, int y_half, int P, int M, int n, const _Float16* svh, void* out,
                                 int out_dt, int64_t out_stride, hipStream_t s) {
    const int waves = M * (n / 128);
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (y_half)
        hipLaunchKernelGGL(lin_had_out_kernel<half_t>, grid, dim3(256), 0, s, (const half_t*)parts, P, M, n, svh, out,
                           out_dt, out_stride);
    else
        hipLaunchKernelGGL(lin_had_out_kernel<float>, grid, dim3(256), 0, s, (const float*)parts, P, M, n, svh, out,
                           out_dt, out_stride);
    return hipGetLastError();
}

hipError_t launch_linear_reconstruct(int K, int cb, const uint32_t* tr, int k, int n, int n0, int n1, _Float16* w,
                                     hipStream_t s) {
    const int k_tiles = k / 16, n_tiles = n / 16, t0 = n0 / 16, t1 = n1 / 16;
    auto launch = [&](auto kern, int ntw) {
        const int waves = k_tiles * ((t1 - t0 + ntw - 1) / ntw);
        hipLaunchKernelGGL(kern, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, tr, k_tiles, n_tiles, t0, t1, w);
    };
    switch (cb * 8 + K) {
        case 16 + 2: launch(lin_reconstruct_kernel<2, 2, half_t>, Geo<2>::NTW); break;
        case 16 + 3: launch(lin_reconstruct_kernel<3, 2, half_t>, Geo<3>::NTW); break;
        case 16 + 4: launch(lin_reconstruct_kernel<4, 2, half_t>, Geo<4>::NTW); break;
        case 16 + 5: launch(lin_reconstruct_kernel<5, 2, half_t>, Geo<5>::NTW); break;
        case 16 + 6: launch(lin_reconstruct_kernel<6, 2, half_t>, Geo<6>::NTW); break;
        case 8 + 4: launch(lin_reconstruct_kernel<4, 1, half_t>, Geo<4>::NTW); break;
        case 8 + 6: launch(lin_reconstruct_kernel<6, 1, half_t>, Geo<6>::NTW); break;
        case 4: launch(lin_reconstruct_kernel<4, 0, half_t>, Geo<4>::NTW); break;
        case 6: launch(lin_reconstruct_kernel<6, 0, half_t>, Geo<6>::NTW); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_linear_had_in_q8(const LinearArgs& a, int8_t* xq, float* sx, int64_t ms, hipStream_t s) {
    const int per_wave = (a.k / 128 + kQ8Waves - 1) / kQ8Waves;
    auto launch = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)(a.S * a.M)), dim3(64 * kQ8Waves), 0, s, a, xq, sx, ms);
    };
    if (per_wave <= 1) launch(lin_had_in_q8_kernel<1>);
    else if (per_wave <= 2) launch(lin_had_in_q8_kernel<2>);
    else if (per_wave <= 4) launch(lin_had_in_q8_kernel<4>);
    else if (per_wave <= 8) launch(lin_had_in_q8_kernel<8>);
    else if (per_wave <= 16) launch(lin_had_in_q8_kernel<16>);
    else launch(lin_had_in_q8_kernel<0>);
    return hipGetLastError();
}

hipError_t launch_linear_reconstruct_q8(int K, const uint32_t* tr, int k, int n, int n0, int n1, int8_t* w,
                                        hipStream_t s) {
    const int k_tiles = k / 16, n_tiles = n / 16, t0 = n0 / 16, t1 = n1 / 16;
    auto launch = [&](auto kern, int ntw) {
        const int waves = k_tiles * ((t1 - t0 + ntw - 1) / ntw);
        hipLaunchKernelGGL(kern, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, tr, k_tiles, n_tiles, t0, t1, w);
    };
    switch (K) {
        case 2: launch(lin_reconstruct_kernel<2, 2, int8_t>, Geo<2>::NTW); break;
        case 3: launch(lin_reconstruct_kernel<3, 2, int8_t>, Geo<3>::NTW); break;
        case 4: launch(lin_reconstruct_kernel<4, 2, int8_t>, Geo<4>::NTW); break;
        case 5: launch(lin_reconstruct_kernel<5, 2, int8_t>, Geo<5>::NTW); break;
        case 6: launch(lin_reconstruct_kernel<6, 2, int8_t>, Geo<6>::NTW); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_linear_had_out_q8(const int32_t* y, const float* sx, float sw, int M, int ng, const _Float16* svh,
                                    void* out, int out_dt, int64_t out_stride, hipStream_t s) {
    const int waves = M * (ng / 128);
    hipLaunchKernelGGL(lin_had_out_q8_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, y, sx, sw, M, ng,
                       svh, out, out_dt, out_stride);
    return hipGetLastError();
}

}  // namespace exl3
