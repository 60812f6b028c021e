// Quantised block formats of the expert bank, shared by host and device code.
//
// Type codes are ggml's enum values so traces stay comparable with llama.cpp
// (sabah/runtime/rt.py:20-23; Q6_K = 14 and Q8_K = 15 are the same enum).
// Geometry follows sabah_rt.cu:2155-2191 for Q8_0/Q5_1/Q4_K/Q5_K/IQ3_S/
// IQ3_XXS/IQ2_S/IQ4_NL/IQ4_XS/Q2_0 and gguf-py quants.py:586-606 for Q6_K
// (ql[128] qh[64] int8 scales[16] fp16 d).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "iq3s_grid.h"
#include "iq_tables.h"

namespace sabah {

enum : int {
    QT_F32 = 0,
    QT_Q5_1 = 7,
    QT_Q8_0 = 8,
    QT_Q8_1 = 9,
    QT_Q4_K = 12,
    QT_Q5_K = 13,
    QT_Q6_K = 14,
    QT_Q8_K = 15,
    QT_IQ3_XXS = 18,
    QT_IQ4_NL = 20,
    QT_IQ3_S = 21,
    QT_IQ2_S = 22,
    QT_IQ4_XS = 23,
    QT_Q2_0 = 42,
};

__host__ __device__ constexpr int block_elems(int qt) {
    return (qt == QT_Q8_0 || qt == QT_Q8_1 || qt == QT_Q5_1 || qt == QT_IQ4_NL) ? 32
         : qt == QT_Q2_0 ? 64
         : (qt == QT_Q4_K || qt == QT_Q5_K || qt == QT_Q6_K || qt == QT_Q8_K || qt == QT_IQ3_S ||
            qt == QT_IQ3_XXS || qt == QT_IQ4_XS || qt == QT_IQ2_S) ? 256 : 0;
}

__host__ __device__ constexpr int block_bytes(int qt) {
    return qt == QT_Q8_0 ? 34
         : qt == QT_Q8_1 ? 36         // fp16 d, fp16 s = d * sum(q), 32 x int8
         : qt == QT_Q5_1 ? 24         // fp16 d, fp16 m, u32 qh, 16 bytes of nibbles
         : qt == QT_Q4_K ? 144
         : qt == QT_Q5_K ? 176        // fp16 d, dmin, 12 bytes of scales / mins, qh[32], qs[128]
         : qt == QT_Q6_K ? 210
         : qt == QT_Q8_K ? 292
         : qt == QT_IQ3_S ? 110
         : qt == QT_IQ3_XXS ? 98      // fp16 d, qs[64] grid indices, 8 x u32 (4 x 7-bit signs, 4-bit scale)
         : qt == QT_IQ4_NL ? 18       // fp16 d, 16 bytes of level nibbles
         : qt == QT_IQ2_S ? 82        // fp16 d, qs[32], signs[32], qh[8], scales[8]
         : qt == QT_IQ4_XS ? 136      // fp16 d, u16 scales_h, scales_l[4], qs[128]
         : qt == QT_Q2_0 ? 18 : 0;    // fp16 d, 16 bytes of 2-bit codes
}

__host__ __device__ inline size_t row_bytes(int qt, int n) {
    const int be = block_elems(qt);
    if (be == 0 || n % be) return 0;
    return (size_t)(n / be) * (size_t)block_bytes(qt);
}

// The activation format ggml's CPU pairs with each weight type (its
// vec_dot_type): q8_0 for Q8_0 and IQ4_NL; q8_K for the K-quants, IQ3_S,
// IQ3_XXS, IQ2_S and IQ4_XS.  Q2_0 takes q8_0, two blocks per weight block
// (ggml's CPU code for Q2_0 is not in the reference: a choice, see the oracle).
__host__ __device__ constexpr int act_type(int qt) {
    return (qt == QT_Q8_0 || qt == QT_IQ4_NL || qt == QT_Q2_0) ? QT_Q8_0
         : qt == QT_Q5_1 ? QT_Q8_1
         : (qt == QT_Q4_K || qt == QT_Q5_K || qt == QT_Q6_K || qt == QT_IQ3_S || qt == QT_IQ3_XXS ||
            qt == QT_IQ4_XS || qt == QT_IQ2_S) ? QT_Q8_K : -1;
}

__host__ __device__ constexpr bool supported_weight_type(int qt) {
    return qt == QT_Q8_0 || qt == QT_Q5_1 || qt == QT_Q4_K || qt == QT_Q5_K || qt == QT_Q6_K || qt == QT_IQ3_S ||
           qt == QT_IQ3_XXS || qt == QT_IQ4_NL ||
           qt == QT_IQ4_XS || qt == QT_IQ2_S || qt == QT_Q2_0;
}

// Expanded IQ3_S codebook entry: byte j = 2*level_j + 1.
__host__ __device__ constexpr uint32_t iq3s_entry(uint16_t lv) {
    return (uint32_t)(2 * ((lv >> 0) & 7) + 1) | ((uint32_t)(2 * ((lv >> 3) & 7) + 1) << 8) |
           ((uint32_t)(2 * ((lv >> 6) & 7) + 1) << 16) | ((uint32_t)(2 * ((lv >> 9) & 7) + 1) << 24);
}

struct Iq3sGrid {
    uint32_t e[512];
};
__host__ __device__ constexpr Iq3sGrid make_iq3s_grid() {
    Iq3sGrid g{};
    for (int i = 0; i < 512; ++i) g.e[i] = iq3s_entry(kIq3sGridLevels[i]);
    return g;
}
// the expanded codebook as device constant memory; kernels copy it into LDS
__constant__ Iq3sGrid kIq3sGridDev = make_iq3s_grid();

__host__ __device__ constexpr Iq3xxsGrid make_iq3xxs_grid() {
    Iq3xxsGrid g{};
    for (int i = 0; i < 256; ++i) g.e[i] = kIq3xxsGridWords[i];
    return g;
}
// the IQ3_XXS codebook (magnitudes 4 .. 62, one per byte) as device constant memory
__constant__ Iq3xxsGrid kIq3xxsGridDev = make_iq3xxs_grid();

struct Iq2sGrid {
    uint32_t w[2048];
};
__host__ __device__ constexpr Iq2sGrid make_iq2s_grid() {
    Iq2sGrid g{};
    for (int i = 0; i < 2048; ++i) g.w[i] = kIq2sGridWords[i];
    return g;
}
// the IQ2_S codebook (two dwords per entry, magnitudes 8 / 25 / 43) as device constant memory
__constant__ Iq2sGrid kIq2sGridDev = make_iq2s_grid();

// ---------------------------------------------------------------------------
// Device-side activation row layout (LDS scratch, never an ABI):
//   qs   int8 chunks of 256 values, chunk c at c * kActChunkStride
//   d    float[kp / QB]      per-block scale (q8_0: the fp16-rounded value)
//   bsum int16[kp / 16]      q8_K: sums of 16 consecutive qs
//        float[kp / 32]      q8_1: s = d * sum of the block's qs (fp16-rounded)
// kp = k rounded up to a multiple of 256; the padding quantises zeros.  The
// 16-byte pad between chunks puts the chunks of one row in different LDS
// banks, so lanes reading different chunks at the same offset do not conflict.
// ---------------------------------------------------------------------------
__host__ __device__ inline size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

constexpr int kActChunkStride = 272;

struct ActLayout {
    int k, at;             // elements, activation type (QT_Q8_0 / QT_Q8_1 / QT_Q8_K)
    size_t off_d, off_bsum, bytes;
    __host__ __device__ ActLayout(int k_, int at_) : k(k_), at(at_) {
        const int qb = block_elems(at_);
        const size_t nchunk = (size_t)((k_ + 255) / 256);
        const size_t kp = nchunk * 256;
        off_d = nchunk * kActChunkStride;
        off_bsum = align16(off_d + sizeof(float) * (kp / (size_t)qb));
        bytes = align16(off_bsum + (at_ == QT_Q8_K ? sizeof(int16_t) * (kp / 16)
                                    : at_ == QT_Q8_1 ? sizeof(float) * (kp / 32) : 0));
    }
};

}  // namespace sabah
