// Device building blocks for EXL3 (mul1 trellis) experts on CDNA4 (gfx950, wave64).
//
// Trellis tile: 16x16 weights of K bits = 8K uint32 words, MSB-first bit stream. Value t (0..255) is the 16-bit window
// ending at bit (t+1)K of the tile stream (circular) and lands at
//     row = 8((t>>1)&1) + 2((t>>3)&3) + (t&1)   (input / k)      col = (t>>5) + 8((t>>2)&1)   (output / n)
// (reference: kernels/moe-a8/exl3_esimd.h:4-14). A "period" is D = K/gcd(K,32) words holding V = 32/gcd(K,32)
// values; a tile has G = 256/V periods. Lanes of a wave own one period each, so every lane decodes the same value
// positions u = 0..V-1 with compile-time shifts.
//
// Codebook mul1 (exl3_esimd.h:40-68): x = s * 0x83DCD12D mod 2^32, h = 1024 + bytesum(x) (its bit pattern is
// 0x6400 + bytesum as fp16, exact), w = RNE_fp16(h * c1 + c2). On gfx950 v_mul_lo_u32 is full rate, so the decode is
// bfe + mul + sad, and two values that share an activation pair go through one v_dot2_f32_f16.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3 {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_bits;

constexpr float kC1 = 0.00676727294921875f;   // fp16 0x1eee
constexpr float kC2 = -10.3828125f;           // fp16 0xc931
constexpr float kRsqrt128 = 0.08838834764831845f;
constexpr uint32_t kMul1 = 0x83DCD12Du;

constexpr int cgcd(int a, int b) { return b == 0 ? a : cgcd(b, a % b); }

template <int K>
struct Geo {
    static constexpr int g = cgcd(K, 32);
    static constexpr int D = K / g;          // words per period
    static constexpr int V = 32 / g;         // values per period
    static constexpr int G = 256 / V;        // periods per tile
    static constexpr int W = 8 * K;          // words per tile
    static constexpr int NTW = 64 / G;       // tiles covered by one wave (one period per lane)
    static_assert(G <= 64, "K too large for one period per lane");
};

// ---- codebook -------------------------------------------------------------------------------------------------------

// raw fp16 bit pattern of h = 1024 + bytesum(s * mul1) in the low 16 bits (s may carry garbage above bit 15 only if
// the caller masks; all callers pass clean 16-bit states)
__device__ __forceinline__ uint32_t cb_raw(uint32_t s) {
    return __builtin_amdgcn_sad_u8(s * kMul1, 0u, 0x6400u);
}
__device__ __forceinline__ half_t cb_h(uint32_t s) {
    return __builtin_bit_cast(half_t, (uint16_t)cb_raw(s));
}
// h of states s0 and s1 as one packed fp16 pair (s0 in the low half) in two instructions after the multiplies:
// v_sad_u8 adds bytesum(s0 * mul1) to 0x6400 in both halves (at most 0x67FC, no carry into the high half), then
// v_sad_hi_u8 adds bytesum(s1 * mul1) << 16
__device__ __forceinline__ uint32_t cb_raw2(uint32_t s0, uint32_t s1) {
    return __builtin_amdgcn_sad_hi_u8(s1 * kMul1, 0u, __builtin_amdgcn_sad_u8(s0 * kMul1, 0u, 0x64006400u));
}
__device__ __forceinline__ half2_t cb_h2(uint32_t s0, uint32_t s1) {
    return __builtin_bit_cast(half2_t, cb_raw2(s0, s1));
}
// bit-exact codebook value: h * c1 + c2 is exact in fp32 (22 significant bits), one rounding to fp16 (RNE)
__device__ __forceinline__ half_t cb_w(uint32_t s) {
    return (half_t)__builtin_fmaf((float)cb_h(s), kC1, kC2);
}
// the same for states s0 and s1 (s0 in the low half) in one v_pk_fma_f16: c1 and c2 are fp16 values and the fused
// multiply-add rounds the exact h * c1 + c2 once (RNE), so each half equals cb_w (no result is subnormal: |w| > 1e-3)
__device__ __forceinline__ half2_t cb_w2(uint32_t s0, uint32_t s1) {
    return __builtin_elementwise_fma(cb_h2(s0, s1), half2_t{(half_t)kC1, (half_t)kC1},
                                     half2_t{(half_t)kC2, (half_t)kC2});
}

// codebooks 3inst (CB 0) and mcg (CB 1) (exl3_esimd.h:69-79): x = s * a + b mod 2^32, m = (x & 0x8FFF8FFF) ^
// 0x3B603B60, w = RNE_fp16(half(m & 0xFFFF) + half(m >> 16)). The mask and xor leave both halves normal with
// magnitude in [1/8, 2), so no subnormal arises in the sum.
template <int CB>
__device__ __forceinline__ uint32_t cb_lcg_m(uint32_t s) {
    static_assert(CB == 0 || CB == 1, "3inst or mcg");
    const uint32_t x = CB == 0 ? s * 89226354u + 64248484u : s * 0xCBAC1FEDu;
    return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
}
// the values of states s0 and s1 (s0 in the low half): v_perm_b32 gathers the two low halves and the two high halves
// of m into one register each, then one v_pk_add_f16 adds them (RNE)
template <int CB>
__device__ __forceinline__ half2_t cb_w2_lcg(uint32_t s0, uint32_t s1) {
    const uint32_t m0 = cb_lcg_m<CB>(s0), m1 = cb_lcg_m<CB>(s1);
    const uint32_t lo = __builtin_amdgcn_perm(m1, m0, 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(m1, m0, 0x07060302u);
    return __builtin_bit_cast(half2_t, lo) + __builtin_bit_cast(half2_t, hi);
}
// the pair a dot product takes for codebook CB: mul1 (CB 2) the raw h (its affine is applied to the dot product by
// the caller), 3inst / mcg the weights themselves
template <int CB>
__device__ __forceinline__ half2_t cb_dot_pair(uint32_t s0, uint32_t s1) {
    if constexpr (CB == 2) return cb_h2(s0, s1);
    else return cb_w2_lcg<CB>(s0, s1);
}

// ---- trellis state extraction -----------------------------------------------------------------------------------------
// Period-relative stream bits: [-32, 0) = previous period's last word, [32j, 32j+32) = word j of the period.
// Every 16-bit window lies either inside one word or inside a funnel F_m = stream bits [32m-16, 32m+16) around a word
// boundary, so after D funnel alignbits every state is one v_bfe_u32 (a clean 16-bit value).

template <int K>
struct Period {
    static constexpr int D = Geo<K>::D;
    uint32_t w[D];       // words of the period
    uint32_t f[D];       // f[m] = stream bits [32m - 16, 32m + 16)
    __device__ __forceinline__ void set(const uint32_t* words, uint32_t prev) {
#pragma unroll
        for (int j = 0; j < D; ++j) w[j] = words[j];
        f[0] = __builtin_amdgcn_alignbit(prev, w[0], 16);
#pragma unroll
        for (int m = 1; m < D; ++m) f[m] = __builtin_amdgcn_alignbit(w[m - 1], w[m], 16);
    }
    // state of value u (compile-time)
    template <int u>
    __device__ __forceinline__ uint32_t state() const {
        constexpr int e = K * (u + 1);                 // window = stream bits [e-16, e)
        constexpr int j = (e - 16) >= 0 ? (e - 16) / 32 : -1;
        constexpr bool in_word = j >= 0 && e <= 32 * j + 32;
        if constexpr (in_word) {
            return __builtin_amdgcn_ubfe(w[j], (uint32_t)(32 * j + 32 - e), 16u);
        } else {
            constexpr int m = (e - 1) / 32;            // boundary 32m lies inside the window
            return __builtin_amdgcn_ubfe(f[m], (uint32_t)(32 * m + 16 - e), 16u);
        }
    }
};

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

// word offset of (tile-row r, tile-col `tile`, period p, plane i) in the checkpoint's natural order: each tile's 8K
// words in stream order, period p = words [p D, p D + D)
template <int K>
__device__ __forceinline__ size_t word_off_nat(int r, int tiles_n, int tile, int p, int i) {
    return ((size_t)r * tiles_n + tile) * Geo<K>::W + p * Geo<K>::D + i;
}

// position of value u of period p inside the 16x16 tile
template <int K>
__host__ __device__ constexpr int val_row(int p, int u) {
    int t = Geo<K>::V * p + u;
    return 8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1);
}
template <int K>
__host__ __device__ constexpr int val_col(int p, int u) {
    int t = Geo<K>::V * p + u;
    return (t >> 5) + 8 * ((t >> 2) & 1);
}

// ---- wave helpers -----------------------------------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// v of lane (lane ^ m) for m = 1, 2, ..., 32 without the LDS crossbar: DPP within 16-lane rows (xor 1, 2: quad
// permutes; xor 4: half-row mirror then quad xor 3; xor 8: row rotate by 8), gfx950 permlane swaps across rows
// (xor 16, 32: swap, then take the half holding the partner). The whole wave must be active.
__device__ __forceinline__ float lane_xor(float v, int m) {
    const int x = __float_as_int(v);
    switch (m) {
        case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));    // quad_perm [1,0,3,2]
        case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));    // quad_perm [2,3,0,1]
        case 4: {
            const int h = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);                // row_half_mirror: ^7
            return __int_as_float(__builtin_amdgcn_mov_dpp(h, 0x1B, 0xF, 0xF, false));        // quad_perm [3,2,1,0]
        }
        case 8: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));   // row_ror:8
        case 16: {
            const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
            return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
        }
        default: {
            const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
            return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += lane_xor(v, m);
    return v;
}

// In-wave unnormalised Sylvester Walsh-Hadamard of 128 values, lane l holding x[2l] (v0) and x[2l+1] (v1).
// Butterflies in the order of exl3_esimd.h:210-220 (h = 1, 2, ..., 64), lower element a + b, upper a - b: the fp32
// results are identical to the sequential restatement.
// Each cross-lane butterfly is one FMA with the lane's sign s (+1 lower, -1 upper), no select: v s + p inside a row
// (v + p, p - v), and across rows the permlane swap's own pair (r0, r1), which is (own, partner) in the lower half and
// (partner, own) in the upper, as r0 + s r1. Each result is the same single rounding of the same two operands.
__device__ __forceinline__ void wave_fwht128(float& v0, float& v1) {
    {
        float a = v0 + v1, b = v0 - v1;
        v0 = a;
        v1 = b;
    }
    const int l = lane_id();
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const float sg = (l & m) ? -1.0f : 1.0f;
        v0 = __builtin_fmaf(v0, sg, lane_xor(v0, m));
        v1 = __builtin_fmaf(v1, sg, lane_xor(v1, m));
    }
    {
        const float sg = (l & 16) ? -1.0f : 1.0f;
        const auto r0 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v0), __float_as_uint(v0), false, false);
        const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v1), __float_as_uint(v1), false, false);
        v0 = __builtin_fmaf(__uint_as_float(r0[1]), sg, __uint_as_float(r0[0]));
        v1 = __builtin_fmaf(__uint_as_float(r1[1]), sg, __uint_as_float(r1[0]));
    }
    {
        const float sg = (l & 32) ? -1.0f : 1.0f;
        const auto r0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v0), false, false);
        const auto r1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v1), __float_as_uint(v1), false, false);
        v0 = __builtin_fmaf(__uint_as_float(r0[1]), sg, __uint_as_float(r0[0]));
        v1 = __builtin_fmaf(__uint_as_float(r1[1]), sg, __uint_as_float(r1[0]));
    }
}

// The same transform over the 16 lanes of a DPP row, lane l holding x[8 (l % 16) + j] in v[j]: butterflies h = 1, 2, 4
// in registers, h = 8 .. 64 across lanes (xor 1, 2, 4, 8 inside the row) as one FMA with the lane's sign (+1 lower,
// -1 upper: v + p and p - v, each rounded once like the add and subtract). Same order and operations as wave_fwht128,
// so the fp32 results are identical; a wave transforms 4 rows at once. The whole wave must be active.
__device__ __forceinline__ void row_fwht128(float (&v)[8]) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
    const int l = lane_id();
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const float sg = (l & m) ? -1.0f : 1.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(v[j], sg, lane_xor(v[j], m));
    }
}

// row_fwht128 up to a sign per lane, in fewer instructions: each cross-lane butterfly is v + s p with the lane's sign
// s, so the partner p is the multiplicand and its DPP move folds into the v_fmac_f32 (the compiler does not fold a DPP
// move into v_fmac_f32, so the stages are written as such). The upper lane of a pair then holds v - p = -(p - v)
// (exactly: rounding to nearest is symmetric), and the two lanes of every later pair carry the same accumulated sign,
// so the result is exactly row_sign() times row_fwht128's. Callers fold row_sign() into the scale they multiply by.
// The whole wave must be active (DPP reads the partner lane unconditionally).
__device__ __forceinline__ float row_sign() {
    return (__builtin_popcount(lane_id() & 15) & 1) ? -1.0f : 1.0f;
}
__device__ __forceinline__ void row_fwht128_signed(float (&v)[8]) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
    const int l = lane_id();
    const float s1 = (l & 1) ? -1.0f : 1.0f, s2 = (l & 2) ? -1.0f : 1.0f;
    const float s4 = (l & 4) ? -1.0f : 1.0f, s8 = (l & 8) ? -1.0f : 1.0f;
    // v[j] += s * v[j] of lane l ^ m. Each block starts with s_nop 1: a DPP source must be written by a VALU at least
    // two wait states before it is read, whatever the compiler placed before the block; inside a block every DPP
    // source was written at least seven instructions earlier.
#define EXL3_FMAC8(CTRL, S)                                                                                      \
    asm("s_nop 1\n\t"                                                                                          \
        "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"                                    \
        "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf"                                          \
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])          \
        : "v"(S))
    EXL3_FMAC8("quad_perm:[1,0,3,2]", s1);                                                      // xor 1
    EXL3_FMAC8("quad_perm:[2,3,0,1]", s2);                                                      // xor 2
    {   // xor 4: the half-row mirror (lane ^ 7) as its own move, then quad_perm [3,2,1,0] (^ 3) in the multiply-add
        float h[8];
        asm("s_nop 1\n\t"
            "v_mov_b32_dpp %0, %8 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %1, %9 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %2, %10 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %3, %11 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %4, %12 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %5, %13 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %6, %14 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %7, %15 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "s_nop 1\n\t"
            "v_fmac_f32_dpp %8, %0, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %9, %1, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %10, %2, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %11, %3, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %12, %4, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %13, %5, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %14, %6, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf\n\t"
            "v_fmac_f32_dpp %15, %7, %16 quad_perm:[3,2,1,0] row_mask:0xf bank_mask:0xf"
            : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(h[4]), "=&v"(h[5]), "=&v"(h[6]), "=&v"(h[7]),
              "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
            : "v"(s4));
    }
    EXL3_FMAC8("row_ror:8", s8);                                                                // xor 8
#undef EXL3_FMAC8
}

// SiLU(g) * u as both expert paths (decode and prefill) compute it, so that one token gets the same fp16 act from
// either: g * rcp(1 + exp(-g)) * u on the hardware exp and reciprocal (__expf is v_exp_f32 of the fp32 product
// -g * log2(e); v_exp_f32 and v_rcp_f32 are each within about 1 ulp in fp32). The reference evaluates
// g / (1 + exp(-g)) * u under -ffast-math SYCL (kernels/moe-a8/exl3_moe.a8.sycl:250). Over every finite fp16 g, with
// any 1-ulp error of the exp and the reciprocal, SiLU(g) stays within 4e-6 relative of the exact value (most of it
// the fp32 rounding of -g * log2(e) at large |g|), and its fp16 rounding is at most one fp16 ulp from the exact
// value's; tests/test_oracle_exl3.py checks both bounds.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

__device__ __forceinline__ float bf16_to_f32(bf16_bits b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ bf16_bits f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);      // round to nearest even (finite inputs)
    return (bf16_bits)(u >> 16);
}
// fp16 of an fp32 value rounded as a step of its own. Written as (half_t)(a * b), the product and the conversion fold
// into one v_fma_mixlo_f16, which rounds the exact product once to fp16; the reference rounds the product to fp32 and
// then to fp16, and the two disagree where the fp32 product lands on an fp16 tie. The empty asm keeps the fp32 value.
__device__ __forceinline__ half_t to_half(float v) {
    asm volatile("" : "+v"(v));
    return (half_t)v;
}

// activation dtypes: 0 fp16, 1 bf16, 2 fp32
__device__ __forceinline__ float ld_act(const void* x, int dt, size_t i) {
    if (dt == 1) return bf16_to_f32(((const bf16_bits*)x)[i]);
    if (dt == 2) return ((const float*)x)[i];
    return (float)((const half_t*)x)[i];
}
// activations i and i + 1 as raw bits (the low 32 for the 16-bit types, all 64 for fp32) from two 32-bit loads that
// are always issued, at any alignment and without a branch: the aligned word holding element i and, when the pair
// reaches into it, the next one (else the same word again, so nothing past the pair is read). act2_cvt converts them
// once they are needed, so that loads issued after these need not wait for them.
__device__ __forceinline__ uint64_t ld_act2_raw(const void* x, int dt, size_t i) {
    const uintptr_t a = (uintptr_t)x + i * (dt == 2 ? 4 : 2);
    const uint32_t* w = (const uint32_t*)(a & ~(uintptr_t)3);
    const unsigned sh = (unsigned)(a & 3) * 8;
    const uint32_t* wn = (dt == 2 || sh) ? w + 1 : w;
    const uint32_t w0 = *w, w1 = *wn;
    return ((((uint64_t)w1) << 32) | w0) >> sh;
}
__device__ __forceinline__ void act2_cvt(uint64_t r, int dt, float& a, float& b) {
    if (dt == 2) {
        a = __uint_as_float((uint32_t)r);
        b = __uint_as_float((uint32_t)(r >> 32));
    } else if (dt == 1) {
        a = bf16_to_f32((bf16_bits)(r & 0xffffu));
        b = bf16_to_f32((bf16_bits)((r >> 16) & 0xffffu));
    } else {
        a = (float)__builtin_bit_cast(half_t, (uint16_t)(r & 0xffffu));
        b = (float)__builtin_bit_cast(half_t, (uint16_t)((r >> 16) & 0xffffu));
    }
}
__device__ __forceinline__ void st_act(void* y, int dt, size_t i, float v) {
    if (dt == 1) ((bf16_bits*)y)[i] = f32_to_bf16(v);
    else if (dt == 2) ((float*)y)[i] = v;
    else ((half_t*)y)[i] = to_half(v);
}

// ---- victim ring claim (experimental/n111-victim-ring/a9.patch:46-65) ------------------------------------------------
// The call's write-backs, in victim order, take the free slots (key < 0) of the ring in circular order from the next
// search position meta[0], each with the next claim number (meta[1] + 1, ...); once no free slot is left the rest are
// dropped and counted (meta[2]); the search position moves past the last slot claimed. This is the order in which the
// reference's serial loop claims, computed with two workgroup scans instead of one slot at a time. scan(v, total)
// is the workgroup's exclusive scan (it contains barriers, so every thread calls this uniformly); rank_slot holds K
// ints of LDS. Returns this thread's ring slot, or -1 (no write-back, or dropped).
template <int NT, typename Scan>
__device__ __forceinline__ int ring_claim(int32_t* meta, int K, int key, int* rank_slot, Scan scan) {
    const int tid = threadIdx.x;
    int nwb;
    const int wbrank = scan(key >= 0 ? 1 : 0, nwb);
    const int p = meta[0], seq0 = meta[1];
    int nfree = 0;
    for (int c0 = 0; c0 < K; c0 += NT) {         // the ring in circular order from p, NT slots at a time
        const int t = c0 + tid;
        int j = p + t;
        j = j >= K ? j - K : j;
        const bool fr = t < K && meta[4 + j] < 0;
        int nf;
        const int r = nfree + scan(fr ? 1 : 0, nf);
        if (fr && r < nwb) rank_slot[r] = j;
        nfree += nf;
    }
    __syncthreads();
    const int nclaim = min(nwb, nfree);
    int slot = -1;
    if (key >= 0 && wbrank < nclaim) {
        slot = rank_slot[wbrank];
        meta[4 + slot] = key;
        meta[4 + K + slot] = seq0 + 1 + wbrank;
    }
    if (tid == 0) {                              // every thread read meta[0] and meta[1] before the first barrier
        const int last = nclaim > 0 ? rank_slot[nclaim - 1] : -1;
        if (nclaim > 0) meta[0] = last + 1 == K ? 0 : last + 1;
        meta[1] = seq0 + nclaim;
        meta[2] += nwb - nclaim;
    }
    return slot;
}

// ---- cross-workgroup exchange ------------------------------------------------------------------------------------------
// Each XCD has a private L2, and an agent-scope fence (__threadfence) writes back and invalidates the whole L2
// (buffer_wbl2 / buffer_inv). Data exchanged between workgroups of one kernel therefore uses agent-scope atomic stores
// and loads (global_store/load ... sc1: written through to / read from the device coherence point) and the producer
// waits for its stores (vmcnt(0)) before the workgroup barrier that precedes the counter increment.
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// sum_i p[i * stride] for i = 0..n-1 in index order, loads issued 16 at a time (one round trip per 16 values)
__device__ __forceinline__ float sum_agent(const float* p, int n, int stride) {
    float acc = 0.f;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = ld_agent(p + (size_t)(i + j) * stride);
#pragma unroll
        for (int j = 0; j < 16; ++j) acc += v[j];
    }
    if (i < n) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = i + j < n ? ld_agent(p + (size_t)(i + j) * stride) : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (i + j < n) acc += v[j];
    }
    return acc;
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ int counter_add(int* c, int v) {
    return __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_reset(int* c) { __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// global-address-space view of a generic pointer (global_load instead of flat_load)
typedef const __attribute__((address_space(1))) uint32_t gu32_t;
__device__ __forceinline__ gu32_t* as_global(const uint32_t* p) { return (gu32_t*)p; }

}  // namespace exl3
