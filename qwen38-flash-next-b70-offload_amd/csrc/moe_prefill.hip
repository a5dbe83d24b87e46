// Prefill MoE (M >= prefill_min_m rows): token sort by expert + grouped GEMMs on MFMA with the EXL3 trellis decoded
// into LDS (reference: moe_prefill a8:792-828, launch_align a8:639-680, GateUpDpasKernel a8:422-545,
// DownDpasKernel a8:548-635, CombineKernel<TO, fp16> a8:371-395).
//
//   align      three small kernels (count per chunk of 1,024 pairs, scan, scatter): pairs sorted by expert in
//              ascending pair order inside an expert (deterministic; wave ballots for in-chunk ranks)
//   xh         input Hadamards xh = fp16(H(fp16(x * suh)) / sqrt(128)) once per (sorted pair, projection), as MFMA
//              products with the +-1 matrix H128 (the column-tile workgroups of an expert all read them)
//   gate/up    one workgroup of 8 waves per (active expert, 128-column block of I), over the expert's rows in passes
//              of 192: the 4 tile-rows x (8 gate + 8 up) tiles of each 64-deep K chunk are decoded once into LDS as
//              the fp16 B operand of v_mfma_f32_32x32x16_f16, the chunk's xh rows staged into LDS with 128-byte row
//              loads (both double-buffered; one barrier per chunk), fp32 accumulation over all of H; epilogue through
//              LDS: g/u Hadamards, SwiGLU, * suh_d, Hadamard -> abuf (fp16), with the reference's rounding points
//   down       one workgroup per (active expert, 256 columns of H), K = I, same decode/MFMA scheme, A = abuf rows;
//              epilogue: output Hadamard * (w * svh_d) -> y (fp16, as the reference's prefill stores it)
//   combine    out[m] = sum_k y[pair_of[m, k]] in k order (fp32), converted to the activation dtype
#include "exl3_common.cuh"
#include "exl3_geom.h"
#include "exl3_kernels.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kAlignChunk = 1024;
constexpr int kPfWaves = 8, kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 192;                    // rows per pass of a GEMM workgroup (6 blocks of 32)
constexpr int kPfRb = kPfRows / 64;             // 32-row blocks per wave (a wave takes the even or the odd blocks)
constexpr int kTileB = 16 * 16 * 2;             // one decoded 16x16 fp16 tile in LDS: [col][k], k-halves swizzled
constexpr int kBRow = 16 * kTileB;              // one tile-row of the 16 tiles (256 columns) of a workgroup
constexpr int kBChunk = 4 * kBRow;              // B of one K chunk (4 tile-rows, K = 64): 32 KB
constexpr int kARow = 64 * 2;                   // one A row of a K chunk (64 fp16), 16-byte pieces swizzled
constexpr int kAProj = kPfRows * kARow;         // A of one projection and K chunk: 24 KB
// double-buffered B and A (gate/up: both projections); the fp32 epilogue tile [64][256] reuses the B buffers
constexpr int pf_lds(int nproj) { return 2 * (kBChunk + nproj * kAProj); }
// the fp32 epilogue tile [64 rows][256 columns] at a row stride of 260 floats: the 16-byte row reads of the epilogues
// (16 lanes per row, 4 rows per wave) then fall on disjoint bank groups in each pair of 8-lane blocks that
// ds_read_b128 serves together (at 256 the pairs (0, 3), (1, 2), ... collide)
constexpr int kEpRow = 260;
// (the tile reaches past the B buffers into the A buffers, both idle between the last chunk and the next pass)
static_assert(pf_lds(2) <= 160 * 1024, "gate/up buffers exceed the LDS of a CU");
static_assert(64 * kEpRow * 4 <= pf_lds(1), "the epilogue tile must fit the LDS of both GEMM kernels");

// ---- block scan helpers (1,024 threads) ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int l = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(v, d, 64);
        if (l >= d) v += t;
    }
    return v;
}
// exclusive scan over the block; tot = block sum. sw: LDS [16 + 1]
__device__ __forceinline__ int block_scan_1024(int v, int* sw, int& tot) {
    const int l = lane_id(), w = threadIdx.x >> 6;
    const int inc = wave_incl_scan(v);
    if (l == 63) sw[w] = inc;
    __syncthreads();
    if (w == 0) {
        const int x = l < 16 ? sw[l] : 0;
        const int xi = wave_incl_scan(x);
        if (l < 16) sw[l] = xi - x;
        if (l == 15) sw[16] = xi;
    }
    __syncthreads();
    const int r = sw[w] + inc - v;
    tot = sw[16];
    __syncthreads();
    return r;
}

// ---- align -----------------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(1024) align_count_kernel(const int32_t* ids, int npairs, int E, int* chunk_cnt) {
    extern __shared__ int hist[];                 // [E]
    for (int e = threadIdx.x; e < E; e += 1024) hist[e] = 0;
    __syncthreads();
    const int i = blockIdx.x * kAlignChunk + threadIdx.x;
    if (i < npairs) atomicAdd(&hist[min(max(ids[i], 0), E - 1)], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 1024) chunk_cnt[(size_t)blockIdx.x * E + e] = hist[e];
}

// per expert (one thread each, E <= 1024): totals, starts, active list, padded starts; chunk counts -> chunk offsets
__global__ void __launch_bounds__(1024) align_scan_kernel(int nchunks, int E, int pad, int* chunk_cnt, AlignOut o) {
    __shared__ int sw[17];
    const int e = threadIdx.x;
    constexpr int kB = 16;                        // chunk counts loaded together (clamped indices: no branch per load)
    int tot = 0;
    if (e < E)
        for (int c0 = 0; c0 < nchunks; c0 += kB) {
            int v[kB];
#pragma unroll
            for (int j = 0; j < kB; ++j) v[j] = chunk_cnt[(size_t)min(c0 + j, nchunks - 1) * E + e];
#pragma unroll
            for (int j = 0; j < kB; ++j) tot += c0 + j < nchunks ? v[j] : 0;
        }
    int all;
    const int st = block_scan_1024(e < E ? tot : 0, sw, all);
    const int act = (e < E && tot > 0) ? 1 : 0;
    int nact;
    const int ai = block_scan_1024(act, sw, nact);
    const int pc = (tot + pad - 1) / pad * pad;
    int ptot;
    const int pst = block_scan_1024(e < E ? pc : 0, sw, ptot);
    if (act) {
        o.act_expert[ai] = e;
        o.act_start[ai] = st;
        o.act_cnt[ai] = tot;
        o.act_pstart[ai] = pst;
    }
    if (e == 0) o.n_act[0] = nact;
    if (o.ord_expert) {
        // the GEMM dispatch order: active experts by descending key = 32-row blocks (capped at 255; two passes rank
        // above one), ties by ascending id. Position = experts with a larger key + lower ids with the same key: ranks
        // inside a wave from ballots, per-(wave, key) counts turned into offsets.
        __shared__ int wk[16 * 256];
        const int l = lane_id(), wv = threadIdx.x >> 6;
        const int key = act ? min((tot + 31) >> 5, 255) : -1;
        for (int i = threadIdx.x; i < 16 * 256; i += 1024) wk[i] = 0;
        __syncthreads();
        uint64_t todo = __ballot(key >= 0);
        int rk = 0;
        while (todo) {
            const int leader = __builtin_ctzll(todo);
            const int kv = __shfl(key, leader, 64);
            const uint64_t m = __ballot(key == kv);
            if (key == kv) rk = __popcll(m & ((1ull << l) - 1));
            if (l == leader) wk[wv * 256 + kv] = __popcll(m);
            todo &= ~m;
        }
        __syncthreads();
        const int kt = 255 - (int)threadIdx.x;    // threads 0..255 own the keys in descending order
        int ck = 0;
        if (kt >= 0)
            for (int w = 0; w < 16; ++w) ck += wk[w * 256 + kt];
        int nsort;
        const int above = block_scan_1024(kt >= 0 ? ck : 0, sw, nsort);
        if (kt >= 0)
            for (int w = 0, run = above; w < 16; ++w) {
                const int c = wk[w * 256 + kt];
                wk[w * 256 + kt] = run;
                run += c;
            }
        __syncthreads();
        if (key >= 0) {
            const int pos = wk[wv * 256 + key] + rk;
            o.ord_expert[pos] = e;
            o.ord_start[pos] = st;
            o.ord_cnt[pos] = tot;
        }
    }
    if (e < E) {                                  // the counts become each chunk's first position of expert e
        int run = st;
        for (int c0 = 0; c0 < nchunks; c0 += kB) {
            int v[kB];
#pragma unroll
            for (int j = 0; j < kB; ++j) v[j] = chunk_cnt[(size_t)min(c0 + j, nchunks - 1) * E + e];
#pragma unroll
            for (int j = 0; j < kB; ++j)
                if (c0 + j < nchunks) {
                    chunk_cnt[(size_t)(c0 + j) * E + e] = run;
                    run += v[j];
                }
        }
    }
}

// positions: chunk offset of the expert + pairs of that expert in earlier waves of the chunk + rank inside the wave
__global__ void __launch_bounds__(1024) align_scatter_kernel(const int32_t* ids, const float* w, int npairs, int topk,
                                                             int E, const int* chunk_off, AlignOut o) {
    extern __shared__ int wh[];                   // [16][E] per-wave counts, then per-wave offsets
    for (int i = threadIdx.x; i < 16 * E; i += 1024) wh[i] = 0;
    __syncthreads();
    const int l = lane_id(), wv = threadIdx.x >> 6;
    const int i = blockIdx.x * kAlignChunk + threadIdx.x;
    const bool valid = i < npairs;
    const int e = valid ? min(max(ids[i], 0), E - 1) : -1;
    uint64_t todo = __ballot(valid);
    int rank = 0;
    while (todo) {
        const int leader = __builtin_ctzll(todo);
        const int ev = __shfl(e, leader, 64);
        const uint64_t m = __ballot(valid && e == ev);
        if (valid && e == ev) rank = __popcll(m & ((1ull << l) - 1));
        if (l == leader) wh[wv * E + ev] = __popcll(m);
        todo &= ~m;
    }
    __syncthreads();
    for (int x = threadIdx.x; x < E; x += 1024) {
        int run = 0;
        for (int q = 0; q < 16; ++q) {
            const int v = wh[q * E + x];
            wh[q * E + x] = run;
            run += v;
        }
    }
    __syncthreads();
    if (valid) {
        const int pos = chunk_off[(size_t)blockIdx.x * E + e] + wh[wv * E + e] + rank;
        o.pair_tok[pos] = i / topk;
        o.pair_w[pos] = w[i];
        o.pair_of[i] = pos;
        if (o.pair_exp) o.pair_exp[pos] = e;
    }
}

hipError_t launch_align(const int32_t* ids, const float* w, int npairs, int topk, int E, int pad, int* chunk_scratch,
                        const AlignOut& o, hipStream_t s) {
    const int nch = npairs > 0 ? (npairs + kAlignChunk - 1) / kAlignChunk : 0;
    if (nch == 0) {                               // no pairs: empty lists, n_act = 0 (no memset: graph-safe)
        hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(1024), 0, s, 0, E, pad, chunk_scratch, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(align_count_kernel, dim3(nch), dim3(1024), E * sizeof(int), s, ids, npairs, E, chunk_scratch);
    hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(1024), 0, s, nch, E, pad, chunk_scratch, o);
    hipLaunchKernelGGL(align_scatter_kernel, dim3(nch), dim3(1024), 16 * E * sizeof(int), s, ids, w, npairs, topk, E,
                       (const int*)chunk_scratch, o);
    return hipGetLastError();
}

// ---- xh pre-pass: input Hadamards as MFMA products with the +-1 matrix H128 ------------------------------------------
// xh[s][pj][kb*128 + n] = fp16(sum_k H[n][k] * fp16(x[tok(s)][kb*128 + k] * suh_pj(e(s))[kb*128 + k]) / sqrt(128)).
// Computed transposed (C^T = H * xt^T) with v_mfma_f32_32x32x16_f16: A = rows n of H, B = 32 pair rows of xt (built in
// registers from x and the pair's expert's suh), so each lane ends with 4 consecutive columns of one pair row per
// accumulator group. H[n][k] = (-1)^popc(n & k) splits over the bits of n and k: with n = 32 nb + n', k = 16 ks + k'
// (n' < 32, k' < 16), popc(n & k) = popc(n' & (16 (ks & 1) + k')) + popc(nb & (ks >> 1)), so the A fragment of
// (nb, ks) is one of two per-lane fragments, negated when popc(nb & (ks >> 1)) is odd: four fragments in registers
// (built once per wave) instead of an H table in LDS. The fp32 sums differ from the butterfly order only in
// rounding. Workgroup of 4 waves per (64 sorted pairs, projection): wave w takes the 32 rows 32 (w & 1) .. and the
// 128-column blocks kb = (w >> 1), (w >> 1) + 2, ... The fp16 results of a block go through LDS ([pair][column]) so
// that 16 lanes store one pair's 256-byte row segment with 16-byte stores.
constexpr int kXhWaves = 4;
constexpr int kXhRow = 128 + 8;                                  // LDS row of one pair's block (halfs, padded)

// 8 consecutive activations as fp32 (exact for every input dtype); DT: 0 fp16, 1 bf16, 2 fp32
template <int DT>
__device__ __forceinline__ void ld_act8(const void* x, size_t i, float (&v)[8]) {
    if constexpr (DT == 2) {
        const float4 a = *(const float4*)((const float*)x + i), b = *(const float4*)((const float*)x + i + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else if constexpr (DT == 1) {
        const uint4 u = *(const uint4*)((const bf16_bits*)x + i);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    } else {
        const half8_t h = *(const half8_t*)((const half_t*)x + i);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)h[j];
    }
}

template <int DT>
__device__ __forceinline__ void xh_blocks(const PrefillArgs& A, half_t (*tbuf)[32 * kXhRow]) {
    const int H = A.g.H, nkb = H / 128;
    const int l = lane_id(), wv = threadIdx.x >> 6;
    half8_t hf[2][2];                                            // [ks & 1][negated]: rows n' = l % 32, k' = 8 (l / 32) + j
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool neg = __popc((l & 31) & (b * 16 + (l >> 5) * 8 + j)) & 1;
            hf[b][0][j] = neg ? (half_t)-1.0f : (half_t)1.0f;
            hf[b][1][j] = neg ? (half_t)1.0f : (half_t)-1.0f;
        }
    // the two projections of a block of 64 pairs run on one XCD (blockIdx b and b + 8), so that the second can read the
    // gathered x rows from that XCD's L2; the grid is rounded up to 16 workgroups
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int pj = slot & 1, blk = (slot >> 1) * 8 + xcd;
    if (blk * 64 >= A.npairs) return;
    // this lane's pair row (B operand column); lanes past the last pair read the last pair, so that no load is
    // conditional and the 16 loads of a block are in flight together (those rows are never stored)
    const int s = min(blk * 64 + (wv & 1) * 32 + (l & 31), A.npairs - 1);
    const size_t xrow = (size_t)A.pair_tok[s] * A.x_stride;
    const half_t* suh = (const half_t*)((const uint8_t*)A.ptrs[A.pair_exp[s]] + (pj ? A.g.off_suh_u : A.g.off_suh_g));
    const int s0 = blk * 64 + (wv & 1) * 32;                    // the wave's 32 pairs
    half_t* tb = tbuf[wv];
    for (int kb = (wv >> 1); kb < nkb; kb += 2) {
        half8_t bx[8];                                           // xt fragments: k = 16 ks + 8 (l / 32) .. + 7
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int k = kb * 128 + ks * 16 + (l >> 5) * 8;
            float xv[8];
            ld_act8<DT>(A.x, xrow + k, xv);
            const half8_t sv = *(const half8_t*)(suh + k);
#pragma unroll
            for (int j = 0; j < 8; ++j) bx[ks][j] = to_half(xv[j] * (float)sv[j]);
        }
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            float16_t acc = float16_t{};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const half8_t ha = hf[ks & 1][__popc(nb & (ks >> 1)) & 1];
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, bx[ks], acc, 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {                        // rows n = 32 nb + 8 q + 4 (l / 32) + 0..3
                const int n = nb * 32 + q * 8 + (l >> 5) * 4;
                typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
                const half4_t hv = half4_t{to_half(acc[4 * q] * kRsqrt128), to_half(acc[4 * q + 1] * kRsqrt128),
                                           to_half(acc[4 * q + 2] * kRsqrt128), to_half(acc[4 * q + 3] * kRsqrt128)};
                *(half4_t*)(tb + (l & 31) * kXhRow + n) = hv;
            }
        }
        // the block's 32 rows x 128 columns: 16 lanes per pair row, 16 bytes each (the wave's own LDS rows)
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int pr = r * 4 + (l >> 4), col = (l & 15) * 8;
            const half8_t v = *(const half8_t*)(tb + pr * kXhRow + col);
            if (s0 + pr < A.npairs) *(half8_t*)(A.xh + ((size_t)(s0 + pr) * 2 + pj) * H + kb * 128 + col) = v;
        }
    }
}

__global__ void __launch_bounds__(64 * kXhWaves) __attribute__((amdgpu_waves_per_eu(4))) prefill_xh_kernel(PrefillArgs A) {
    __shared__ __align__(16) half_t tbuf[kXhWaves][32 * kXhRow]; // per wave: [pair][column] of one block
    // the block loop per activation dtype (no dtype branch between a block's loads)
    if (A.x_dt == 1) xh_blocks<1>(A, tbuf);
    else if (A.x_dt == 2) xh_blocks<2>(A, tbuf);
    else xh_blocks<0>(A, tbuf);
}

// ---- LDS layouts of one K chunk ----------------------------------------------------------------------------------------
// B: tile j of tile-row kt at kt * kBRow + j * kTileB, column c of the tile at 32 c, its k-half h (k = 8 h .. 8 h + 7)
// in the 16-byte slot h ^ (j & 1). On gfx950 a ds_read_b128 serves the 8-lane blocks (0, 3), (1, 2), (4, 7) and (5, 6)
// of a wave together, and a block of 8 consecutive columns at 32-byte spacing covers the even or the odd 16-byte bank
// groups of a 256-byte row, as its slot parity says. In a B-fragment read the block of lanes 8 b .. 8 b + 7 holds tile
// b >> 1 & 1, k-half b >> 2 and columns 8 (b & 1) .. + 7, so its parity is (b >> 2) ^ (b >> 1 & 1), which differs in
// each of those pairs of blocks: one pass per 16 lanes (a parity that also flipped with c >> 3 made every pair collide,
// half the read rate). A decoder store's 8-lane blocks alternate tiles, hence parities.
__device__ __forceinline__ int b_slot(int tile, int c, int h) {
    return tile * kTileB + c * 32 + ((h ^ (tile & 1)) << 4);
}
// A: row r of the chunk at r * kARow, its 16-byte piece j (k = 8 j .. 8 j + 7) in slot j ^ ((r >> 1) & 7): 16 rows of one
// piece (an A-fragment read) and 2 rows of 8 pieces (a staging store) each hit 16 distinct slots.
__device__ __forceinline__ int a_slot(int r, int j) { return r * kARow + ((j ^ ((r >> 1) & 7)) << 4); }

// ---- decode of one K chunk (4 tile-rows x 16 tiles) into LDS ----------------------------------------------------------
// The 16 tiles of a workgroup: local tile j lives at global tile column tcol(j). Period q of the chunk:
// tile-row q / (16 G), local tile (q / G) % 16, period p = q % G; G consecutive lanes hold one tile's periods, so the
// circular previous word of a period comes from the neighbouring lane. Value u of period p (t = V p + u) lies in column
// (V p >> 5) + 8 ((u >> 2) & 1) and k-half (u >> 1) & 1, at position 2 ((V p >> 3) & 3) + 2 (u >> 3) + (u & 1) of that
// half: a period fills V / 4 consecutive k of 4 (column, k-half) slots, so it is stored as 4 vector writes of V / 2 bytes.
template <int K>
struct ChunkDecoder {
    using GM = Geo<K>;
    static constexpr int G = GM::G, D = GM::D, V = GM::V;
    static constexpr int PER = 4 * 16 * G / kPfThreads;     // periods per thread per chunk (1, 2 or 4)
    static constexpr int E = V / 4;                         // values per (column, k-half) slot of a period
    static_assert(PER >= 1 && 4 * 16 * G == PER * kPfThreads, "chunk periods must split evenly");
    uint32_t wd[PER][D];

    __device__ __forceinline__ static int tile_of(int q) { return (q / G) % 16; }
    __device__ __forceinline__ static int trow_of(int q) { return q / (16 * G); }

    template <typename TCol>
    __device__ __forceinline__ static void load(uint32_t (&w)[PER][D], const uint32_t* tr, int tiles_n, int kt0,
                                                TCol tcol) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int q = threadIdx.x + j * kPfThreads;
            const int p = q % G;
#pragma unroll
            for (int i = 0; i < D; ++i)
                w[j][i] = __builtin_nontemporal_load(as_global(tr) +
                                                     word_off<K>(kt0 + trow_of(q), tiles_n, tcol(tile_of(q)), p, i));
        }
    }

    // slot (column 8 ci + (V p >> 5), k-half kh): values u = 8 (e >> 1) + 4 ci + 2 kh + (e & 1), e = 0 .. E - 1; the
    // values e = 2 f and 2 f + 1 are states u and u + 1, decoded as one pair
    typedef _Float16 hv_t __attribute__((ext_vector_type(E)));
    typedef uint32_t hp_t __attribute__((ext_vector_type(E / 2)));
    template <int ci, int kh, int... f>
    __device__ __forceinline__ static hv_t slot_vals(const Period<K>& P, std::integer_sequence<int, f...>) {
        return __builtin_bit_cast(
            hv_t, hp_t{__builtin_bit_cast(uint32_t, cb_w2(P.template state<(f << 3) | (ci << 2) | (kh << 1)>(),
                                                          P.template state<(f << 3) | (ci << 2) | (kh << 1) | 1>()))...});
    }

    // this thread's periods of the chunk (the previous word of each comes from the neighbouring lane)
    __device__ __forceinline__ void prep(Period<K> (&P)[PER]) const {
        const int l = lane_id();
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int q = threadIdx.x + j * kPfThreads;
            const int p = q % G;
            const int src = (l / G) * G + (p + G - 1) % G;
            P[j].set(wd[j], (uint32_t)__shfl((int)wd[j][D - 1], src, 64));
        }
    }
    // slot s (= 2 ci + kh) of every period: a quarter of the chunk's values of this thread
    template <int s>
    __device__ __forceinline__ static void slot(const Period<K> (&P)[PER], hv_t (&o)[PER][4]) {
        constexpr auto es = std::make_integer_sequence<int, E / 2>{};
#pragma unroll
        for (int j = 0; j < PER; ++j) o[j][s] = slot_vals<(s >> 1), (s & 1)>(P[j], es);
    }
    // the chunk's values of this thread: 4 slots per period (16 VGPRs for every K)
    __device__ __forceinline__ void decode(hv_t (&o)[PER][4]) const {
        Period<K> P[PER];
        prep(P);
        slot<0>(P, o);
        slot<1>(P, o);
        slot<2>(P, o);
        slot<3>(P, o);
    }

    __device__ __forceinline__ static void store(const hv_t (&o)[PER][4], uint8_t* buf) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int q = threadIdx.x + j * kPfThreads;
            const int p = q % G, tile = tile_of(q);
            uint8_t* tb = buf + trow_of(q) * kBRow + tile * kTileB + ((V * p) >> 5) * 32 + 4 * ((V * p >> 3) & 3);
            const int sw = (tile & 1) << 4;
            *(hv_t*)(tb + (0 ^ sw)) = o[j][0];
            *(hv_t*)(tb + (16 ^ sw)) = o[j][1];
            *(hv_t*)(tb + 8 * 32 + (0 ^ sw)) = o[j][2];
            *(hv_t*)(tb + 8 * 32 + (16 ^ sw)) = o[j][3];
        }
    }

    // decode and store slot by slot (fewer live registers than decode + store)
    __device__ __forceinline__ void decode_store(uint8_t* buf) const {
        Period<K> P[PER];
        prep(P);
        constexpr auto es = std::make_integer_sequence<int, E / 2>{};
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int q = threadIdx.x + j * kPfThreads;
            const int p = q % G, tile = tile_of(q);
            uint8_t* tb = buf + trow_of(q) * kBRow + tile * kTileB + ((V * p) >> 5) * 32 + 4 * ((V * p >> 3) & 3);
            const int sw = (tile & 1) << 4;
            *(hv_t*)(tb + (0 ^ sw)) = slot_vals<0, 0>(P[j], es);
            *(hv_t*)(tb + (16 ^ sw)) = slot_vals<0, 1>(P[j], es);
            *(hv_t*)(tb + 8 * 32 + (0 ^ sw)) = slot_vals<1, 0>(P[j], es);
            *(hv_t*)(tb + 8 * 32 + (16 ^ sw)) = slot_vals<1, 1>(P[j], es);
        }
    }
};

// ---- the GEMM core shared by gate/up and down -------------------------------------------------------------------------
// C[rows][256] (rows <= 192) over nchunks K chunks of 64: wave w takes the 32-row blocks rb = (w >> 2) + 2 j (j < 3) and
// the 64 columns 64 (w & 3) .. + 63 (2 fragments of 32), so the two waves of a SIMD (w, w + 4) share its matrix core
// evenly. A (the workgroup's rows of NPROJ fp16 matrices, projection of wave w = (w & 3) >> 1 when NPROJ = 2) and B
// (the decoded trellis) of a chunk sit in LDS, double-buffered, one barrier per chunk. In the loop, waves 0-3 multiply
// chunk c first and then produce chunk c + 1 (decode B, store the staged A, issue the loads for chunk c + 2) while
// waves 4-7 produce first and multiply after.

// A of a K chunk staged through registers: group g = wave + 8 i covers projection g / 24, rows 8 (g % 24) .. + 7 with
// 16-byte loads (lane: row + l / 8, piece l % 8, so 8 lanes read one row's 128 bytes) and 16-byte LDS stores into the
// swizzled slots; rows at or beyond `rows` are zero
template <int NPROJ>
struct AStage {
    static constexpr int NL = NPROJ * kPfRows / 64;          // 16-byte loads per lane per chunk (8 rows x 128 B each)
    uint4 v[NL];
    // rows at or past `rows` read as zero through the buffer descriptor's range (num_records = rows * lda halfs, in
    // bytes: row rows - 1 of the last projection still lies inside it, row `rows` of the first does not), so the loads
    // carry no branch per row and nothing past the pass's rows is read
    __device__ __forceinline__ void load(const half_t* a, size_t lda, size_t proj_off, int rows, int k0) {
        const int l = lane_id(), wv = threadIdx.x >> 6;
        const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a), (short)0, rows * (int)lda * 2,
                                                            0x00020000);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int g = wv + 8 * i, pj = g / (kPfRows / 8), r = (g % (kPfRows / 8)) * 8 + (l >> 3);
            const int off = (pj * (int)proj_off + r * (int)lda + k0 + (l & 7) * 8) * 2;
            const auto t = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
            v[i] = make_uint4(t[0], t[1], t[2], t[3]);
        }
    }
    __device__ __forceinline__ void store(uint8_t* buf, int nrb) const {
        const int l = lane_id(), wv = threadIdx.x >> 6;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int g = wv + 8 * i, pj = g / (kPfRows / 8), r8 = (g % (kPfRows / 8)) * 8;
            if (r8 < nrb * 32) *(uint4*)(buf + pj * kAProj + a_slot(r8 + (l >> 3), l & 7)) = v[i];
        }
    }
};

template <int K, int NPROJ, typename TCol>
__device__ __forceinline__ void gemm_core(const uint32_t* tr, int tiles_n, int nchunks, TCol tcol, const half_t* a,
                                          size_t lda, size_t proj_off, int rows, uint8_t* lds,
                                          float16_t (&acc)[kPfRb][2]) {
    using Dec = ChunkDecoder<K>;
    const int wv = threadIdx.x >> 6, l = lane_id();
    const int rpar = wv >> 2, q = wv & 3, proj = NPROJ == 2 ? (q >> 1) : 0;
    const int nrb = (rows + 31) >> 5;
    const bool mfma_first = rpar == 0;
#pragma unroll
    for (int j = 0; j < kPfRb; ++j) acc[j][0] = acc[j][1] = float16_t{};
    uint8_t* const b0 = lds;
    uint8_t* const a0 = lds + 2 * kBChunk;
    Dec dec;
    AStage<NPROJ> ast;
    // this lane's B-fragment offsets (columns 64 q + l % 32 and + 32, k-half l / 32)
    const int n = q * 64 + (l & 31);
    const int boff0 = b_slot(n >> 4, n & 15, l >> 5), boff1 = b_slot((n + 32) >> 4, n & 15, l >> 5);
    // the wave's live row blocks j < nj (rb = rpar + 2 j < nrb), as a compile-time count: no branch per block, so the
    // fragment reads of a K step go out together
    const int nj = (nrb - rpar + 1) >> 1;
    auto mfma_n = [&](auto NJ, int cur) {
        constexpr int kNj = decltype(NJ)::value;
        const uint8_t* bb = b0 + cur * kBChunk;
        const uint8_t* ab = a0 + cur * (NPROJ * kAProj) + proj * kAProj;
        if constexpr (NPROJ == 1 && K <= 3) {
            // down at K <= 3 (VGPRs to spare; K = 4 would spill): the fragments of K step ks + 1 are read before the
            // MFMAs of step ks, so each step's MFMAs wait only for reads issued one step earlier
            half8_t fb[2][2], fa[2][kNj];
            auto rd = [&](int ks, int st) {
                fb[st][0] = *(const half8_t*)(bb + ks * kBRow + boff0);
                fb[st][1] = *(const half8_t*)(bb + ks * kBRow + boff1);
#pragma unroll
                for (int j = 0; j < kNj; ++j)
                    fa[st][j] = *(const half8_t*)(ab + a_slot((rpar + 2 * j) * 32 + (l & 31), 2 * ks + (l >> 5)));
            };
            rd(0, 0);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if (ks + 1 < 4) rd(ks + 1, (ks + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < kNj; ++j) {
                    acc[j][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ks & 1][j], fb[ks & 1][0], acc[j][0], 0, 0, 0);
                    acc[j][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ks & 1][j], fb[ks & 1][1], acc[j][1], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            return;
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            // all fragment reads of the K step first (the fence keeps them ahead of the MFMAs)
            const half8_t f0 = *(const half8_t*)(bb + ks * kBRow + boff0);
            const half8_t f1 = *(const half8_t*)(bb + ks * kBRow + boff1);
            half8_t fa[kNj];
#pragma unroll
            for (int j = 0; j < kNj; ++j)
                fa[j] = *(const half8_t*)(ab + a_slot((rpar + 2 * j) * 32 + (l & 31), 2 * ks + (l >> 5)));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < kNj; ++j) {
                acc[j][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[j], f0, acc[j][0], 0, 0, 0);
                acc[j][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[j], f1, acc[j][1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto mfma = [&](int cur) {
        // the multiplying wave issues ahead of the producing wave of its SIMD while its MFMAs last
        __builtin_amdgcn_s_setprio(1);
        switch (nj) {
            case 3: mfma_n(std::integral_constant<int, 3>{}, cur); break;
            case 2: mfma_n(std::integral_constant<int, 2>{}, cur); break;
            case 1: mfma_n(std::integral_constant<int, 1>{}, cur); break;
            default: break;
        }
        __builtin_amdgcn_s_setprio(0);
    };
    auto produce = [&](int c) {                   // chunk c + 1 into its buffers, loads of chunk c + 2
        if (c + 1 < nchunks) {
            dec.decode_store(b0 + ((c + 1) & 1) * kBChunk);
            ast.store(a0 + ((c + 1) & 1) * (NPROJ * kAProj), nrb);
        }
        if (c + 2 < nchunks) {
            Dec::load(dec.wd, tr, tiles_n, 4 * (c + 2), tcol);
            ast.load(a, lda, proj_off, rows, (c + 2) * 64);
        }
    };
    Dec::load(dec.wd, tr, tiles_n, 0, tcol);
    ast.load(a, lda, proj_off, rows, 0);
    produce(-1);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        if (mfma_first) {
            mfma(c & 1);
            produce(c);
        } else {
            produce(c);
            mfma(c & 1);
        }
        __syncthreads();
    }
}

// 32-row blocks 2 g (waves 0-3) and 2 g + 1 (waves 4-7) -> LDS fp32 [64 rows][256 columns]
__device__ __forceinline__ void stash_acc(const float16_t (&acc)[2], float* ep) {
    const int l = lane_id(), wv = threadIdx.x >> 6, rpar = wv >> 2, q = wv & 3;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = rpar * 32 + (i & 3) + 8 * (i >> 2) + 4 * (l >> 5);
            ep[row * kEpRow + q * 64 + cb * 32 + (l & 31)] = acc[cb][i];
        }
}

// workgroup -> (position a of the dispatch order, column block): the nblk workgroups of an expert share blockIdx % 8,
// i.e. one XCD and its L2, which serves the expert's A rows to all of them. Workgroups are dispatched in blockIdx
// order, so the experts with the most rows (two passes first) start first, dealt round-robin over the XCDs, and the
// last workgroups of the launch are the shortest.
__device__ __forceinline__ void pf_block(int nblk, int& a, int& blk) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    a = (slot / nblk) * 8 + xcd;
    blk = slot % nblk;
}

template <int K>
__global__ void __launch_bounds__(kPfThreads) prefill_gateup_kernel(PrefillArgs A) {
    __shared__ __align__(16) uint8_t lds[pf_lds(2)];
    const int I = A.g.I, H = A.g.H, nbn = I / 128;
    int a, nb;
    pf_block(nbn, a, nb);
    if (a >= A.n_act[0]) return;
    const int e = A.ord_expert[a], s0 = A.ord_start[a], cnt = A.ord_cnt[a];
    const uint8_t* base = (const uint8_t*)A.ptrs[e];
    const int wv = threadIdx.x >> 6, l = lane_id();
    const int tiles_n = 2 * I / 16;
    auto tcol = [nb, I](int j) { return j < 8 ? nb * 8 + j : I / 16 + nb * 8 + (j - 8); };
    const half_t* svg = (const half_t*)(base + A.g.off_svh_g);
    const half_t* svu = (const half_t*)(base + A.g.off_svh_u);
    const half_t* sud = (const half_t*)(base + A.g.off_suh_d);
    float* ep = (float*)lds;
    const int cb8 = nb * 128 + (l & 15) * 8;      // this lane's 8 columns of the block (16-lane row layout)
    for (int r0 = 0; r0 < cnt; r0 += kPfRows) {
        const int rows = min(kPfRows, cnt - r0);
        float16_t acc[kPfRb][2];
        // A = xh rows of both projections: xh[(s, pj)][H], row stride 2H, projection offset H
        gemm_core<K, 2>((const uint32_t*)base, tiles_n, H / 64, tcol, A.xh + (size_t)(s0 + r0) * 2 * H, 2 * (size_t)H,
                        (size_t)H, rows, lds, acc);
        const half8_t hg = *(const half8_t*)(svg + cb8), hu = *(const half8_t*)(svu + cb8);
        const half8_t hd = *(const half8_t*)(sud + cb8);
#pragma unroll
        for (int m = 0; m < kPfRb; ++m) {
            if (m * 64 >= rows) break;
            stash_acc(acc[m], ep);
            __syncthreads();
            // 4 rows per wave pass, 16 lanes per row; rows past `rows` are transformed (every lane takes part in the
            // cross-lane butterflies) but not stored
            for (int r4 = wv * 4; r4 < 64; r4 += 4 * kPfWaves) {
                const int rr = r4 + (l >> 4), row = m * 64 + rr;
                const float* er = ep + rr * kEpRow + (l & 15) * 8;
                float g[8], u[8], av[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    g[j] = er[j];
                    u[j] = er[128 + j];
                }
                row_fwht128_signed(g);
                row_fwht128_signed(u);
                const float rs = row_sign() * kRsqrt128;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float gj = (float)to_half(g[j] * rs * (float)hg[j]);
                    const float uj = (float)to_half(u[j] * rs * (float)hu[j]);
                    const float aj = (float)to_half(silu_mul(gj, uj));
                    av[j] = (float)to_half(aj * (float)hd[j]);
                }
                row_fwht128_signed(av);
                half8_t o;
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = to_half(av[j] * rs);
                if (row < rows) *(half8_t*)(A.abuf + (size_t)(s0 + r0 + row) * I + cb8) = o;
            }
            __syncthreads();
        }
    }
}

template <int K>
__global__ void __launch_bounds__(kPfThreads) prefill_down_kernel(PrefillArgs A) {
    __shared__ __align__(16) uint8_t lds[pf_lds(1)];
    const int I = A.g.I, H = A.g.H, ntn = H / 256;
    int a, nt;
    pf_block(ntn, a, nt);
    if (a >= A.n_act[0]) return;
    const int e = A.ord_expert[a], s0 = A.ord_start[a], cnt = A.ord_cnt[a];
    const uint8_t* base = (const uint8_t*)A.ptrs[e];
    const int wv = threadIdx.x >> 6, l = lane_id();
    const int tiles_n = H / 16;
    auto tcol = [nt](int j) { return nt * 16 + j; };
    const half_t* svd = (const half_t*)(base + A.g.off_svh_d);
    float* ep = (float*)lds;
    for (int r0 = 0; r0 < cnt; r0 += kPfRows) {
        const int rows = min(kPfRows, cnt - r0);
        float16_t acc[kPfRb][2];
        gemm_core<K, 1>((const uint32_t*)(base + A.g.gu_bytes), tiles_n, I / 64, tcol, A.abuf + (size_t)(s0 + r0) * I,
                        (size_t)I, 0, rows, lds, acc);
        // 16-lane row layout: lanes 0-31 one row, 32-63 the next; lanes 16-31 and 48-63 the second 128 columns. The
        // lane's 8 output-column scales and the routing weights of the wave's rows are loaded ahead of the rows'
        // Hadamards (no global load inside the row loop)
        const int hb = (l >> 4) & 1, cb8 = nt * 256 + hb * 128 + (l & 15) * 8;
        const half8_t hs = *(const half8_t*)(svd + cb8);
        constexpr int kPass = 64 / (2 * kPfWaves);   // wave passes per 64-row group
#pragma unroll
        for (int m = 0; m < kPfRb; ++m) {
            if (m * 64 >= rows) break;
            float pw[kPass];
#pragma unroll
            for (int i = 0; i < kPass; ++i) {
                const int row = m * 64 + 2 * (wv + kPfWaves * i) + (l >> 5);
                pw[i] = A.pair_w[s0 + r0 + min(row, rows - 1)];
            }
            stash_acc(acc[m], ep);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kPass; ++i) {
                const int rr = 2 * (wv + kPfWaves * i) + (l >> 5), row = m * 64 + rr;
                const float* er = ep + rr * kEpRow + hb * 128 + (l & 15) * 8;
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = er[j];
                row_fwht128_signed(v);                       // the DPP-folded transform, as in the gate/up epilogue
                const float sc = row_sign() * kRsqrt128 * pw[i];
                half8_t o;
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = to_half(v[j] * sc * (float)hs[j]);
                if (row < rows) *(half8_t*)(A.y + (size_t)(s0 + r0 + row) * H + cb8) = o;
            }
            __syncthreads();
        }
    }
}

// out[m][h] = sum over k (in order) of y[pair_of[m topk + k]][h]; 8 columns per thread. Up to kCombMax picks: all
// pick positions, then all rows' loads go out before the sum (a loop would wait for each position and each row in
// turn); more picks take the loop.
constexpr int kCombMax = 16;
// the picks' rows of one token, 8 columns, loaded together (picks past topk repeat the last one and are not summed)
template <int KM>
__device__ __forceinline__ void comb_rows(const PrefillArgs& A, int m, int topk, int H, int h0, float (&acc)[8]) {
    int pos[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) pos[k] = A.pair_of[m * topk + min(k, topk - 1)];
    half8_t v[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) v[k] = *(const half8_t*)(A.y + (size_t)pos[k] * H + h0);
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < topk)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += (float)v[k][j];
}
__global__ void __launch_bounds__(256) prefill_combine_kernel(PrefillArgs A) {
    const int m = blockIdx.x, H = A.g.H, topk = A.topk;
    // one 16-byte store per 8 outputs when the row start allows it (16-bit outputs, 8-aligned offsets)
    const bool vec = A.x_dt != 2 && (A.out_stride & 7) == 0 && ((uintptr_t)A.out & 15) == 0;
    for (int h0 = threadIdx.x * 8; h0 < H; h0 += 256 * 8) {
        float acc[8] = {};
        if (topk <= 10) {
            comb_rows<10>(A, m, topk, H, h0, acc);
        } else if (topk <= kCombMax) {
            comb_rows<kCombMax>(A, m, topk, H, h0, acc);
        } else {
            for (int k = 0; k < topk; ++k) {
                const int pos = A.pair_of[m * topk + k];
                const half8_t v = *(const half8_t*)(A.y + (size_t)pos * H + h0);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] += (float)v[j];
            }
        }
        const size_t oo = (size_t)m * A.out_stride + h0;
        if (vec) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[j] = A.x_dt == 1 ? (uint32_t)f32_to_bf16(acc[2 * j]) | ((uint32_t)f32_to_bf16(acc[2 * j + 1]) << 16)
                                   : (uint32_t)__builtin_bit_cast(uint16_t, (half_t)acc[2 * j]) |
                                         ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)acc[2 * j + 1]) << 16);
            *(uint4*)((uint16_t*)A.out + oo) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) st_act(A.out, A.x_dt, oo + j, acc[j]);
        }
    }
}

size_t align_scratch_bytes(int npairs, int E) {
    return (size_t)((npairs + kAlignChunk - 1) / kAlignChunk) * E * 4;
}

size_t prefill_workspace_bytes(int M, int H, int I, int topk, int E) {
    const size_t np = (size_t)M * topk, A = std::min<size_t>(np, (size_t)E);
    const size_t nch = (np + kAlignChunk - 1) / kAlignChunk;
    return align256((7 * A + 1) * 4) + 3 * align256(np * 4) + align256(np * 4) + align256(nch * E * 4) +
           align256(np * 2 * H * 2) + align256(np * I * 2) + align256(np * H * 2);
}

hipError_t launch_prefill(PrefillArgs a, int E, void* ws, hipStream_t s) {
    const int np = a.npairs, H = a.g.H, I = a.g.I;
    const size_t A = std::min(np, E);
    uint8_t* p = (uint8_t*)ws;
    auto take = [&p](size_t n) { uint8_t* q = p; p += align256(n); return q; };
    AlignOut o;
    int* act = (int*)take((7 * A + 1) * 4);
    o.act_expert = act;
    o.act_start = act + A;
    o.act_cnt = act + 2 * A;
    o.act_pstart = act + 3 * A;
    o.n_act = act + 4 * A;
    o.ord_expert = act + 4 * A + 1;
    o.ord_start = o.ord_expert + A;
    o.ord_cnt = o.ord_start + A;
    o.pair_tok = (int*)take((size_t)np * 4);
    o.pair_of = (int*)take((size_t)np * 4);
    o.pair_exp = (int*)take((size_t)np * 4);
    o.pair_w = (float*)take((size_t)np * 4);
    int* chunk = (int*)take((size_t)((np + kAlignChunk - 1) / kAlignChunk) * E * 4);
    a.xh = (half_t*)take((size_t)np * 2 * H * 2);
    a.abuf = (half_t*)take((size_t)np * I * 2);
    a.y = (half_t*)take((size_t)np * H * 2);
    a.ord_expert = o.ord_expert;
    a.ord_start = o.ord_start;
    a.ord_cnt = o.ord_cnt;
    a.n_act = o.n_act;
    a.pair_tok = o.pair_tok;
    a.pair_w = o.pair_w;
    a.pair_of = o.pair_of;
    a.pair_exp = o.pair_exp;
    hipError_t e = launch_align(a.ids, a.w, np, a.topk, E, 1, chunk, o, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prefill_xh_kernel, dim3((unsigned)((2 * ((np + 63) / 64) + 15) / 16 * 16)), dim3(64 * kXhWaves), 0,
                       s, a);
    const unsigned A8 = (unsigned)((A + 7) / 8 * 8);   // workgroups of an expert share blockIdx % 8
    const dim3 ggu(A8 * (unsigned)(I / 128)), gdn(A8 * (unsigned)(H / 256));
    switch (a.g.K) {
        case 2:
            hipLaunchKernelGGL(prefill_gateup_kernel<2>, ggu, dim3(kPfThreads), 0, s, a);
            hipLaunchKernelGGL(prefill_down_kernel<2>, gdn, dim3(kPfThreads), 0, s, a);
            break;
        case 3:
            hipLaunchKernelGGL(prefill_gateup_kernel<3>, ggu, dim3(kPfThreads), 0, s, a);
            hipLaunchKernelGGL(prefill_down_kernel<3>, gdn, dim3(kPfThreads), 0, s, a);
            break;
        case 4:
            hipLaunchKernelGGL(prefill_gateup_kernel<4>, ggu, dim3(kPfThreads), 0, s, a);
            hipLaunchKernelGGL(prefill_down_kernel<4>, gdn, dim3(kPfThreads), 0, s, a);
            break;
        default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace exl3
