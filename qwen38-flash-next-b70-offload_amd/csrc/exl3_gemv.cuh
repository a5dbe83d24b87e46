// The fused dequant-GEMV pieces shared by the MoE decode kernel and the dense EXL3 linear: the per-period
// accumulation over the raw codebook integers, the bit-exact dequant store and the 8 x 4-tile wave GEMV.
#pragma once
#include "exl3_common.cuh"

namespace exl3 {

// one period of one tile-row: xv[a][qq] holds activation rows (8a + 2q, 8a + 2q + 1), q = (qb + qq) & 3. Values u and
// u + 1 (u even) are the rows of one activation pair in the same column, so one v_dot2_f32_f16 takes both.
template <int K, int NQ, int u>
__device__ __forceinline__ void accum_period(const Period<K>& P, const half2_t (&xv)[2][NQ], float (&acc)[2]) {
    if constexpr (u < Geo<K>::V) {
        static_assert(u % 2 == 0 && Geo<K>::V % 2 == 0, "values are taken in pairs");
        const half2_t h = cb_h2(P.template state<u>(), P.template state<u + 1>());
        acc[(u >> 2) & 1] = __builtin_amdgcn_fdot2(h, xv[(u >> 1) & 1][u >> 3], acc[(u >> 2) & 1], false);
        accum_period<K, NQ, u + 2>(P, xv, acc);
    }
}

// accum_period split in two: the period's raw h pairs decoded ahead of its activations (h[u / 2] for values u, u + 1),
// then the same v_dot2_f32_f16 chain over them once the activations are known
template <int K, int u>
__device__ __forceinline__ void decode_period(const Period<K>& P, half2_t* h) {
    if constexpr (u < Geo<K>::V) {
        h[u >> 1] = cb_h2(P.template state<u>(), P.template state<u + 1>());
        decode_period<K, u + 2>(P, h);
    }
}
template <int K, int NQ, int u>
__device__ __forceinline__ void dot_period(const half2_t* h, const half2_t (&xv)[2][NQ], float (&acc)[2]) {
    if constexpr (u < Geo<K>::V) {
        acc[(u >> 2) & 1] = __builtin_amdgcn_fdot2(h[u >> 1], xv[(u >> 1) & 1][u >> 3], acc[(u >> 2) & 1], false);
        dot_period<K, NQ, u + 2>(h, xv, acc);
    }
}

// the same for MR activation rows at once: each pair of codebook values is decoded once and multiplied into every row
// (codebook CB: mul1 as raw h, 3inst / mcg as the weights, see cb_dot_pair)
template <int K, int NQ, int MR, int u, int CB = 2>
__device__ __forceinline__ void accum_period_mr(const Period<K>& P, const half2_t (&xv)[MR][2][NQ],
                                                float (&acc)[MR][2]) {
    if constexpr (u < Geo<K>::V) {
        const half2_t h = cb_dot_pair<CB>(P.template state<u>(), P.template state<u + 1>());
#pragma unroll
        for (int m = 0; m < MR; ++m)
            acc[m][(u >> 2) & 1] = __builtin_amdgcn_fdot2(h, xv[m][(u >> 1) & 1][u >> 3], acc[m][(u >> 2) & 1], false);
        accum_period_mr<K, NQ, MR, u + 2, CB>(P, xv, acc);
    }
}

// bit-exact store of one period's values (row/col of value u depend on the period for K != 3), decoded in pairs as
// the prefill decoder does, so that the exhaustive dequant checks cover both halves of cb_w2 (cb_w2_lcg for the
// 3inst / mcg codebooks, CB 0 / 1)
template <int K, int u, int CB = 2>
__device__ __forceinline__ void dequant_store(const Period<K>& P, int p, _Float16* o, size_t n_out) {
    if constexpr (u < Geo<K>::V) {
        half2_t w;
        if constexpr (CB == 2) w = cb_w2(P.template state<u>(), P.template state<u + 1>());
        else w = cb_w2_lcg<CB>(P.template state<u>(), P.template state<u + 1>());
        o[(size_t)val_row<K>(p, u) * n_out + val_col<K>(p, u)] = w.x;
        o[(size_t)val_row<K>(p, u + 1) * n_out + val_col<K>(p, u + 1)] = w.y;
        dequant_store<K, u + 2, CB>(P, p, o, n_out);
    }
}

// GEMV of 8 tile-rows x 4 tile-columns per wave (gate/up): one PLANAR4 group, whose 4 tile-columns share every
// 128-byte line of words. Tile tau = pass * NTW + j of the wave's 32 is (tile-row tau / 4, tile-column tau % 4), so a
// lane keeps NCQ = max(1, 4 / NTW) column pairs over all passes.
template <int K>
struct Gemv4 {
    using GM = Geo<K>;
    static constexpr int G = GM::G, D = GM::D, V = GM::V, NTW = GM::NTW, L = 32 / V;
    static constexpr int NQ = V / 8;
    static constexpr int NPS = 32 / NTW;                 // passes
    static constexpr int NCQ = NTW >= 4 ? 1 : 4 / NTW;   // column pairs per lane

    uint32_t wd[NPS][D];

    __device__ __forceinline__ static int trow(int ps, int j) { return (ps * NTW + j) >> 2; }
    __device__ __forceinline__ static int tcol(int ps, int j) { return (ps * NTW + j) & 3; }

    __device__ __forceinline__ void load(const uint32_t* tr, int tiles_n, int rt0, int ct0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int ps = 0; ps < NPS; ++ps)
#pragma unroll
            for (int i = 0; i < D; ++i)
                wd[ps][i] = __builtin_nontemporal_load(as_global(tr) +
                                                       word_off<K>(rt0 + trow(ps, j), tiles_n, ct0 + tcol(ps, j), p, i));
    }

    // the same words from a matrix in the checkpoint's natural order (the dense linear)
    __device__ __forceinline__ void load_nat(const uint32_t* tr, int tiles_n, int rt0, int ct0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int ps = 0; ps < NPS; ++ps)
#pragma unroll
            for (int i = 0; i < D; ++i)
                wd[ps][i] = __builtin_nontemporal_load(
                    as_global(tr) + word_off_nat<K>(rt0 + trow(ps, j), tiles_n, ct0 + tcol(ps, j), p, i));
    }

    __device__ __forceinline__ void write_through(uint32_t* trd, int tiles_n, int rt0, int ct0) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int ps = 0; ps < NPS; ++ps)
#pragma unroll
            for (int i = 0; i < D; ++i) trd[word_off<K>(rt0 + trow(ps, j), tiles_n, ct0 + tcol(ps, j), p, i)] = wd[ps][i];
    }

    // victim write-back at this wave's word positions (see Gemv8::copy_old), one pass at a time
    __device__ __forceinline__ void copy_old(const uint32_t* slot, uint32_t* host, int tiles_n, int rt0, int ct0) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll 1
        for (int ps = 0; ps < NPS; ++ps) {
            uint32_t old[D];
            const int rt = rt0 + trow(ps, j), ct = ct0 + tcol(ps, j);
#pragma unroll
            for (int i = 0; i < D; ++i) old[i] = slot[word_off<K>(rt, tiles_n, ct, p, i)];
            wait_stores();
#pragma unroll
            for (int i = 0; i < D; ++i) host[word_off<K>(rt, tiles_n, ct, p, i)] = old[i];
        }
    }

    // xq: the wave's 128-row block, [tile-row][8] half2
    __device__ __forceinline__ void compute(const half2_t* xq, float (&acc)[NCQ][2]) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
        const int qb = ((V * p) >> 3) & 3;
#pragma unroll
        for (int ps = 0; ps < NPS; ++ps) {
            const uint32_t prev = (uint32_t)__shfl((int)wd[ps][D - 1], src_lane, 64);
            Period<K> P;
            P.set(wd[ps], prev);
            const half2_t* xr = xq + trow(ps, j) * 8;
            half2_t xv[2][NQ];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int qq = 0; qq < NQ; ++qq) xv[a][qq] = xr[4 * a + ((qb + qq) & 3)];
            accum_period<K, NQ, 0>(P, xv, acc[ps % NCQ]);
        }
    }

    // compute() for MR activation rows: xq = [MR][64] half2, row m's 128-row block at xq + 64 m; codebook CB
    template <int MR, int CB = 2>
    __device__ __forceinline__ void compute_mr(const half2_t* xq, float (&acc)[MR][NCQ][2]) const {
        const int l = lane_id();
        const int p = l % G, j = l / G;
        const int src_lane = j * G + ((p + G - 1) % G);
        const int qb = ((V * p) >> 3) & 3;
#pragma unroll
        for (int ps = 0; ps < NPS; ++ps) {
            const uint32_t prev = (uint32_t)__shfl((int)wd[ps][D - 1], src_lane, 64);
            Period<K> P;
            P.set(wd[ps], prev);
            half2_t xv[MR][2][NQ];
            float t[MR][2];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const half2_t* xr = xq + m * 64 + trow(ps, j) * 8;
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int qq = 0; qq < NQ; ++qq) xv[m][a][qq] = xr[4 * a + ((qb + qq) & 3)];
                t[m][0] = acc[m][ps % NCQ][0];
                t[m][1] = acc[m][ps % NCQ][1];
            }
            accum_period_mr<K, NQ, MR, 0, CB>(P, xv, t);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                acc[m][ps % NCQ][0] = t[m][0];
                acc[m][ps % NCQ][1] = t[m][1];
            }
        }
    }

    // sum the lanes sharing column pair q (L within a tile, and the tile-rows of one pass when NTW > 4); true for the
    // lane owning it, col0 = its column of h = 0 within the 64-column group (h = 1 is col0 + 8)
    __device__ __forceinline__ static bool reduce(float (&acc)[2], int q, int& col0) {
        const int l = lane_id();
        const int p = l % G, j = l / G;
#pragma unroll
        for (int mm = 1; mm < L; mm <<= 1) {
            acc[0] += lane_xor(acc[0], mm);
            acc[1] += lane_xor(acc[1], mm);
        }
#pragma unroll
        for (int mm = 4 * G; mm < 64; mm <<= 1) {
            acc[0] += lane_xor(acc[0], mm);
            acc[1] += lane_xor(acc[1], mm);
        }
        col0 = tcol(q, j) * 16 + ((V * p) >> 5);
        return j < 4 && (p % L) == 0;
    }
};

}  // namespace exl3
