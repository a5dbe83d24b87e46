// Kernel argument structs and host-side launchers shared by the HIP translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_geom.h"

namespace exl3 {

constexpr int kMaxPairs = 1024;     // pairs (rows x top-k) of one decode call
constexpr int kMaxRows = 256;       // rows of one decode call
constexpr int kMaxExperts = 1024;   // experts per layer (one ensure work-item per expert)
constexpr int kMaxI = 4096;         // intermediate size of the decode kernels (abuf staged in LDS)
// ensure inside the layer kernel (one 512-thread workgroup): its limits
constexpr int kEnsRegSlots = 32;    // slot_last values held in registers per thread: S <= 512 * 32
constexpr int kEnsMaxP = 64;        // picks (one per lane of wave 0)
constexpr int kEnsMaxE = 512;       // experts (one per thread)
constexpr int kVictimRingMax = 256; // victim ring slots (the claim's rank table lives in the ensure's 256-int LDS scratch)

constexpr int kVictimChunkBytes = 64 * 1024;   // bytes of a victim slot copied by one workgroup

struct VictimArgs {
    const int32_t* vict; const int64_t* host_base; int64_t slot_base; int64_t blob; int64_t hstride; int E;
    uint8_t* ram_res; int chunk_bytes;
    const int64_t* vaddr;                          // write-back target of victim i [E] (written by the ensure)
};

struct EnsureArgs {
    int32_t* ids; float* w; int P;                 // picks (masked in place)
    int layer, E, S;
    int64_t* ptrs_all; int32_t* slot_of; int32_t* slot_key; int32_t* slot_last; int32_t* tick;
    const int64_t* host_base; int64_t slot_base; int64_t blob; int64_t hstride;
    int64_t* fill_all; int32_t* fill_list; int max_fill;
    const uint8_t* ram_res; int32_t* ring; int ring_cap; const int32_t* safe;   // tier (null ram_res: off)
    int32_t* vict;                                 // victim list [1 + 2E] or null
    int64_t* vict_addr;                            // with vict: the write-back target of victim i [E] (0: none)
    // record pool of the RAM tier (host_addr null: fixed records at host_base[layer] + e * hstride)
    int64_t* host_addr;                            // host record address of every key [L * E] (stale when not in RAM)
    const int64_t* wbq;                            // free records for this step's write-backs [wbq_cap]
    int32_t* wbq_state;                            // [0] records taken, [1 + i] key written back into wbq[i],
                                                   // [1 + wbq_cap] write-backs dropped (no record left)
    int wbq_cap;
    // victim ring (vr_meta null: off; needs vict and vict_addr): write-backs go to ring slots in device memory and the
    // host drains them to RAM later. vr_meta int32 [4 + 2 vr_K]: [0] next search position, [1] claims made, [2]
    // write-backs dropped (ring full), [3] vr_K, then key[vr_K] (-1: free, else the key awaiting its drain) and
    // seq[vr_K] (the claim number of that key); vr_sel [E]: the ring slot of victim i (-1: none); slots of blob bytes
    int32_t* vr_meta; int32_t* vr_sel; int64_t vr_base; int vr_K;
    int32_t* log; int64_t log_cap;                 // decision log (debug) or null: [count, records...]; log_cap:
                                                   // int32 words after the count (a record is written if it fits)
    int64_t* pair_ptr;                             // out: blob pointer of every post-mask pick [P] (or null)
    int32_t* pair_own;                             // out (ensure inside the layer kernel): 1 if pick i is the first
                                                   // pick of its post-mask expert [P] (or null)
    int32_t* pf_slot;                              // prefetch mode when set: tick not advanced, no fill_all; the
                                                   // slot of each assigned expert (fill_list order) [max_fill]
    int32_t* host_plan;                            // plan mode (with pf_slot): [seq, n, T, layer, e[E], s[E]] in
                                                   // pinned host memory for the copy worker; claimed slots pinned
    int32_t* plan_seq;                             // [n_layers] plans published per layer
    int32_t* pend;                                 // [n_layers][kPendStride] pending plans: n, seq, T, e[16], s[16]
    const int32_t* done_seq;                       // [n_layers] last plan whose copies finished (copy engine)
    int n_layers;                                  // commit finished plans first when pend and n_layers > 0
};
constexpr int kPendStride = 35;                    // pend record: n, seq, T, e[16], s[16]
constexpr int kPlanMax = 16;                       // experts per copy-engine plan

struct DecodeArgs {
    const void* x; int x_dt; int64_t x_stride;     // activations [M, H], dt 0 = fp16, 1 = bf16
    const int32_t* ids; const float* w;            // [M * topk] (post-mask when cached)
    int M, topk, npairs, E;
    const int64_t* ptrs;                           // per-layer blob pointer table [E]
    const int64_t* pair_ptr;                       // blob pointer per pair (written by ensure) or null
    const int64_t* fill;                           // per-layer write-through targets [E] (0 = none) or null
    int64_t* commit_ptrs;                          // cache commit: ptrs[e] = fill[e] for e in fill_list
    int64_t* commit_fill;
    const int32_t* fill_list;                      // [1 + E]
    uint64_t* xpart;                               // tagged gate/up sums [npairs][H/1024 slices][2I] (exchange buffer)
    uint64_t* xy;                                  // tagged y of every pick [npairs][H] (exchange buffer)
    uint64_t* xstart;                              // started word of every gate/up and down workgroup (exchange buffer)
    int n_gu;                                      // gate/up workgroups
    void* out; int64_t out_stride;                 // [M, H], same dtype as x
    BlobGeom g;
    VictimArgs va;                                 // victim write-back (cached calls with victims on)
    int n_vict_wg, vict_chunks;                    // victim-copy workgroups (first in the grid) and chunks per victim
    int fused;                                     // 1: workgroup 0 runs the cache's ensure (ens) inside the launch
    int vict_inline;                               // 1: the writers of a miss copy the victim's old bytes themselves
    EnsureArgs ens;
};

// token sort (reference launch_align a8:639-680): pairs sorted by expert, ascending pair index inside an expert
struct AlignOut {
    int* act_expert; int* act_start; int* act_cnt; int* act_pstart; int* n_act;   // [A], [A], [A], [A], [1]
    int* pair_tok; int* pair_of; float* pair_w;                                    // [npairs] each
    int* pair_exp;                                                                  // expert of each sorted pair or null
    // the active experts again in GEMM dispatch order (descending 32-row block count, ties by ascending id), or null
    int* ord_expert; int* ord_start; int* ord_cnt;                                  // [A] each
};

struct PrefillArgs {
    const void* x; int x_dt; int64_t x_stride;     // activations [M, H]
    const int32_t* ids; const float* w;            // [M * topk]
    int M, topk, npairs;
    const int64_t* ptrs;                           // per-layer blob pointer table [E]
    const int* ord_expert; const int* ord_start; const int* ord_cnt; const int* n_act;   // GEMM dispatch order
    const int* pair_tok; const float* pair_w; const int* pair_of; const int* pair_exp;
    _Float16* xh;                                  // [npairs (sorted)][2][H] input Hadamards (gate, up)
    _Float16* abuf;                                // [npairs (sorted)][I]
    _Float16* y;                                   // [npairs (sorted)][H], routing weight applied
    void* out; int64_t out_stride;                 // [M, H], dtype of x
    BlobGeom g;
};

constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// the dense EXL3 linear (linear.hip): out[M, n] = svh * H(sum_k xh[shard of n][m][k] W[k][n]) / sqrt 128
constexpr int kLinMaxRows = 8;       // rows of the fused small-M path
struct LinearArgs {
    const void* x; int x_dt; int64_t x_stride;     // activations [M, k]
    int M, k, n, S;                                // rows, input and output features, shards
    const uint32_t* tr;                            // trellis words [k/16][n/16][8K], checkpoint (natural) order
    const _Float16* suh;                           // [S][k]
    const _Float16* svh;                           // [n]
    const int32_t* shard_of_nb;                    // [n/128]
    _Float16* xh;                                  // [S][M][k] (the large-M path's input Hadamards)
    uint64_t* part;                                // [P][M][n] tagged partial sums over the K-slices: zero on
                                                   // entry, left zero
    int P;                                         // K-slices (4 blocks of 128 rows each)
    int* status;                                   // device status words (a timed-out poll adds 1 to [0])
    int* const* status_host;                       // the device word holding their host mirror's address (or null)
};
hipError_t launch_linear_had_in(const LinearArgs& a, hipStream_t s);
// the fused small-M linear (M <= kLinMaxRows): input Hadamards, dequant-GEMV and output Hadamard in one launch;
// codebook cb: 2 mul1 (K = 2..6), 1 mcg or 0 3inst (K = 4, 6)
hipError_t launch_linear_small(int K, int cb, const LinearArgs& a, void* out, int out_dt, int64_t out_stride,
                               hipStream_t s);
// out = svh * H(sum of P parts) / sqrt 128; parts fp32 (y_half 0) or one fp16 matrix (y_half 1, P 1)
hipError_t launch_linear_had_out(const void* parts, int y_half, int P, int M, int n, const _Float16* svh, void* out,
                                 int out_dt, int64_t out_stride, hipStream_t s);
// W[k][n1 - n0] fp16 (the codebook's weights) of tile-columns [n0/16, n1/16) of a natural-order trellis
hipError_t launch_linear_reconstruct(int K, int cb, const uint32_t* tr, int k, int n, int n0, int n1, _Float16* w,
                                     hipStream_t s);
// the W8A8 route: xq int8 [S][ms][k] and sx fp32 [S][ms] (row stride ms >= M); int8 mul1 weights of columns
// [n0, n1); out[:, group] = svh * H(y * sx * sw) / sqrt 128 for y int32 [M][ng] of one shard group
hipError_t launch_linear_had_in_q8(const LinearArgs& a, int8_t* xq, float* sx, int64_t ms, hipStream_t s);
hipError_t launch_linear_reconstruct_q8(int K, const uint32_t* tr, int k, int n, int n0, int n1, int8_t* w,
                                        hipStream_t s);
hipError_t launch_linear_had_out_q8(const int32_t* y, const float* sx, float sw, int M, int ng, const _Float16* svh,
                                    void* out, int out_dt, int64_t out_stride, hipStream_t s);
static inline int linear_kslices(int k) { return (k / 128 + 3) / 4; }
// small-M workspace: the tagged partial sums [P][M][n] (64-bit words)
static inline size_t linear_workspace_bytes(int M, int k, int n) {
    return align256((size_t)linear_kslices(k) * M * n * 8);
}

// decode.hip
hipError_t launch_moe_layer(int K, const DecodeArgs& a, hipStream_t s);
int read_status(int* out, hipStream_t s);
hipError_t status_address(void** p);
hipError_t status_host_slot(void** p);           // device address of the word holding the host mirror's address
hipError_t set_status_mirror(int* host_word);
hipError_t launch_dequant(int K, const uint32_t* tr, _Float16* out, int k_tiles, int n_tiles, hipStream_t s);
// cache.hip
hipError_t launch_ensure(const EnsureArgs& a, hipStream_t s);
// prefetch (moe_prefetch a8:1194-1222): ensure in prefetch mode, then copy every assigned expert from its host record
// (host_base[layer] + e * hstride) into its slot (slot_base + s * sstride, `copy_bytes` bytes) and repoint ptrs_all
hipError_t launch_prefetch(const EnsureArgs& a, int64_t sstride, int64_t copy_bytes, hipStream_t s);
// the copies and the commit of a cached call outside the decode kernel, after its ensure (a: the ensure's arguments;
// blob: bytes of the layer's blob; max_n: an upper bound of the call's fills)
hipError_t launch_cached_fills(const EnsureArgs& a, int64_t blob, int max_n, uint8_t* ram_res, hipStream_t s);
hipError_t launch_scatter_flags(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n, hipStream_t s);
hipError_t launch_table_update(int64_t* ptrs_all, int32_t* slot_of, int32_t* slot_key, int32_t* slot_last,
                               const int64_t* rec, int64_t n, hipStream_t s);
struct TierCopy { const uint8_t* src; uint8_t* dst; int64_t n; };   // n bytes, device -> pinned host
struct TierCopies { TierCopy c[4]; int n; };
struct TierRing { const int32_t* ring; int64_t cap, from; int32_t* mirror; };  // ring null: no mirroring
// record pool of the RAM tier: the step's address updates (key, address) applied to host_addr and ptrs_all, then the
// write-back queue: state [2 + cap] copied to the pinned mirror, the next step's records installed, the state cleared
struct TierPool {
    const int64_t* upd; int64_t n_upd; int64_t* host_addr; int64_t* ptrs_all;   // upd: pinned [2 n_upd]
    const int32_t* slot_of;                        // ptrs_all of a key in an HBM slot keeps the slot
    const int64_t* next; int64_t* wbq; int32_t* state; int32_t* mirror; int cap;  // next: pinned [cap]; wbq null: off
};
hipError_t launch_tier_exchange(uint8_t* flags, int64_t n_flags, const int32_t* packed, int64_t n_diff,
                                const TierRing& rg, const TierCopies& cp, const TierPool& pl, hipStream_t s);
// prefill.hip
hipError_t launch_align(const int32_t* ids, const float* w, int npairs, int topk, int E, int pad, int* chunk_scratch,
                        const AlignOut& o, hipStream_t s);
size_t align_scratch_bytes(int npairs, int E);
size_t prefill_workspace_bytes(int M, int H, int I, int topk, int E);
hipError_t launch_prefill(PrefillArgs a, int E, void* ws, hipStream_t s);

// 1024-row slices of H of the decode gate/up workgroups (one 128-row block per wave; H is a multiple of 128)
__host__ __device__ static inline int gu_kslices(int H) { return (H + 1023) / 1024; }

// workspace of a decode call (bytes, 256-aligned parts): the blob pointer of every pick
constexpr size_t decode_workspace_bytes(int npairs, int H, int I) {
    (void)H;
    (void)I;
    return align256((size_t)npairs * 8);
}
// tagged words a decode call exchanges between workgroups (library-owned buffer, zeroed when allocated)
static inline int decode_gu_workgroups(int npairs, int H, int I) { return npairs * 4 * (I / 128) * gu_kslices(H); }
static inline size_t decode_exchange_words(int npairs, int H, int I) {
    return (size_t)npairs * ((size_t)gu_kslices(H) * 2 * I + H) + decode_gu_workgroups(npairs, H, I) +
           (size_t)npairs * (H / 128);
}

}  // namespace exl3
