// Expert blob geometry shared by host and device code.
// Blob (one contiguous region per expert; reference kernels/moe-a8/exl3_moe.a8.sycl:3-13, 42-54):
//   gate|up trellis uint32 [H/16][2I/16][8K] (PLANAR4)  | down trellis uint32 [I/16][H/16][8K] (PLANAR4) |
//   fp16 suh_g[H] suh_u[H] svh_g[I] svh_u[I] suh_d[I] svh_d[H]
#pragma once
#include <stdint.h>

namespace exl3 {

struct BlobGeom {
    int H, I, K;
    int64_t gu_bytes, d_bytes, off_suh_g, off_suh_u, off_svh_g, off_svh_u, off_suh_d, off_svh_d, blob;
};

static inline BlobGeom blob_geom(int H, int I, int K) {
    BlobGeom g;
    g.H = H; g.I = I; g.K = K;
    const int64_t W = 8 * K;
    g.gu_bytes = (int64_t)(H / 16) * (2 * I / 16) * W * 4;
    g.d_bytes = (int64_t)(I / 16) * (H / 16) * W * 4;
    g.off_suh_g = g.gu_bytes + g.d_bytes;
    g.off_suh_u = g.off_suh_g + 2 * (int64_t)H;
    g.off_svh_g = g.off_suh_u + 2 * (int64_t)H;
    g.off_svh_u = g.off_svh_g + 2 * (int64_t)I;
    g.off_suh_d = g.off_svh_u + 2 * (int64_t)I;
    g.off_svh_d = g.off_suh_d + 2 * (int64_t)I;
    g.blob = g.off_svh_d + 2 * (int64_t)H;
    return g;
}

}  // namespace exl3
