// Per-format decoding of one 32-element "item" of a quantised row staged in
// LDS, into packed 8-bit integers plus the item's integer scales.  The same
// item decoder feeds both the integer dot products (sdot4 against q8
// activations) and the dequantiser, so the dequantiser's bit-exact comparison
// with ggml dequantize_row_* also certifies the bits the dot kernels read.
//
// Field layouts (byte offsets inside a block):
//   Q8_0  (34 B / 32):  d f16 @0, qs int8[32] @2                 (sabah_rt.cu:2537-2545)
//   Q4_K  (144 B/256):  d @0, dmin @2, scales[12] @4, qs[128] @16 (sabah_rt.cu:2462-2485)
//   Q6_K  (210 B/256):  ql[128] @0, qh[64] @128, int8 sc[16] @192, d @208 (quants.py:586-606)
//   IQ3_S (110 B/256):  d @0, qs[64] @2, qh[8] @66, signs[32] @74, scales[4] @106
//                       (sabah_rt.cu:2618-2647, quants.py:1132-1159)
#pragma once
#include "quant_formats.h"

namespace sabah {

// ---- LDS byte access ------------------------------------------------------
__device__ inline uint32_t lds_u8(const uint8_t* s, uint32_t off) { return s[off]; }
__device__ inline uint32_t lds_u16(const uint8_t* s, uint32_t off) {
    return *reinterpret_cast<const uint16_t*>(s + off);   // off is even for every field read
}
__device__ inline uint32_t lds_dw(const uint8_t* s, uint32_t off4) {
    return *reinterpret_cast<const uint32_t*>(s + off4);
}
// n consecutive dwords starting at any byte offset (reads n+1 aligned dwords;
// tiles are padded by 16 bytes so the last read stays inside the allocation)
template <int N>
__device__ inline void lds_read_unaligned(const uint8_t* s, uint32_t off, uint32_t (&out)[N]) {
    const uint32_t a = off & ~3u, sh = off & 3u;
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) w[i] = lds_dw(s, a + 4 * i);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

__device__ inline float f16_bits_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// ---- decoded item ----------------------------------------------------------
// v[8]: the item's 32 weights as packed int8 (IQ3_S, Q8_0: signed values;
//       Q4_K: nibbles 0..15; Q6_K: unsigned 6-bit 0..63, offset by 32 in the math)
// s0/s1: integer scales (IQ3_S: 2*scale+1; Q4_K: 6-bit scale, 6-bit min;
//        Q6_K: int8 scales of the item's two 16-element halves; Q8_0: unused)
struct Item {
    uint32_t v[8];
    int s0, s1;
};

// ---- IQ3_S -----------------------------------------------------------------
// Element e = 32*ib + 4*g + j of a super-block: magnitude = byte j of
// grid[qs[8*ib+g] | bit g of qh[ib] << 8], negated when bit (4*(g&1)+j) of
// signs[4*ib + g/2] is set; sub-block scale 2*nibble+1 from scales[ib/2].
__device__ inline Item decode_iq3s(const uint8_t* s, uint32_t blk, int ib, const uint32_t* grid) {
    Item it;
    uint32_t qs[2], sg[1];
    lds_read_unaligned<2>(s, blk + 2 + 8 * ib, qs);
    lds_read_unaligned<1>(s, blk + 74 + 4 * ib, sg);
    const uint32_t qh = lds_u8(s, blk + 66 + ib);
    const uint32_t sc = lds_u8(s, blk + 106 + (ib >> 1));
    it.s0 = 2 * (int)((sc >> (4 * (ib & 1))) & 15u) + 1;
    it.s1 = 0;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t lo = (qs[g >> 2] >> (8 * (g & 3))) & 0xFFu;
        const uint32_t idx = lo | (((qh >> g) & 1u) << 8);
        const uint32_t mag = grid[idx];
        const uint32_t s4 = (sg[0] >> (4 * g)) & 15u;
        const uint32_t t = (s4 * 0x00204081u) & 0x01010101u;   // sign bit j -> bit 8j
        const uint32_t m = t * 0xFFu;                           // 0x00 / 0xFF per byte
        it.v[g] = (mag ^ m) + t;                                // per-byte negate, no carries (mag >= 1)
    }
    return it;
}

// ---- Q4_K ------------------------------------------------------------------
// 6-bit scale/min of sub-block j from the 12 packed bytes (get_scale_min_k4).
__device__ inline void q4k_scale_min(const uint8_t* s, uint32_t blk, int j, int& sc, int& mn) {
    const uint32_t q = blk + 4;
    if (j < 4) {
        sc = (int)(lds_u8(s, q + j) & 63u);
        mn = (int)(lds_u8(s, q + j + 4) & 63u);
    } else {
        sc = (int)((lds_u8(s, q + j + 4) & 0xFu) | ((lds_u8(s, q + j - 4) >> 6) << 4));
        mn = (int)((lds_u8(s, q + j + 4) >> 4) | ((lds_u8(s, q + j) >> 6) << 4));
    }
}
// Sub-block j (elements 32j..32j+31): nibbles of qs[32*(j/2) .. +32], low for
// even j, high for odd j.
__device__ inline Item decode_q4k(const uint8_t* s, uint32_t blk, int j) {
    Item it;
    uint32_t q[8];
    lds_read_unaligned<8>(s, blk + 16 + 32 * (j >> 1), q);
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) it.v[i] = (q[i] >> sh) & 0x0F0F0F0Fu;
    q4k_scale_min(s, blk, j, it.s0, it.s1);
    return it;
}

// ---- Q6_K ------------------------------------------------------------------
// Item j (elements 32j..32j+31) sits in half h = j/4 at quarter s = j%4:
// low 4 bits from ql[64h + 32*(s&1) + l] (nibble s>>1), high 2 bits from
// qh[32h + l] bits 2s..2s+1.  Scales sc[2j], sc[2j+1] cover its two 16-halves.
__device__ inline Item decode_q6k(const uint8_t* s, uint32_t blk, int j) {
    Item it;
    const int h = j >> 2, q = j & 3;
    uint32_t ql[8], qh[8];
    lds_read_unaligned<8>(s, blk + 64 * h + 32 * (q & 1), ql);
    lds_read_unaligned<8>(s, blk + 128 + 32 * h, qh);
    const int nsh = 4 * (q >> 1), hsh = 2 * q;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        it.v[i] = ((ql[i] >> nsh) & 0x0F0F0F0Fu) | (((qh[i] >> hsh) & 0x03030303u) << 4);
    it.s0 = (int)(int8_t)lds_u8(s, blk + 192 + 2 * j);
    it.s1 = (int)(int8_t)lds_u8(s, blk + 192 + 2 * j + 1);
    return it;
}

// ---- Q8_0 ------------------------------------------------------------------
__device__ inline Item decode_q8_0(const uint8_t* s, uint32_t blk) {
    Item it;
    lds_read_unaligned<8>(s, blk + 2, it.v);
    it.s0 = it.s1 = 0;
    return it;
}

// ---- generic dispatch --------------------------------------------------------
// Item p of a row whose first byte is at LDS offset `row`.
template <int QT>
__device__ inline Item decode_item(const uint8_t* s, uint32_t row, int p, const uint32_t* grid) {
    if constexpr (QT == QT_IQ3_S) return decode_iq3s(s, row + 110u * (uint32_t)(p >> 3), p & 7, grid);
    if constexpr (QT == QT_Q4_K) return decode_q4k(s, row + 144u * (uint32_t)(p >> 3), p & 7);
    if constexpr (QT == QT_Q6_K) return decode_q6k(s, row + 210u * (uint32_t)(p >> 3), p & 7);
    if constexpr (QT == QT_Q8_0) return decode_q8_0(s, row + 34u * (uint32_t)p);
}

// fp16 block scale(s) of the block holding item p
template <int QT>
__device__ inline float block_d(const uint8_t* s, uint32_t row, int p) {
    if constexpr (QT == QT_IQ3_S) return f16_bits_to_f32(lds_u16(s, row + 110u * (uint32_t)(p >> 3)));
    if constexpr (QT == QT_Q4_K) return f16_bits_to_f32(lds_u16(s, row + 144u * (uint32_t)(p >> 3)));
    if constexpr (QT == QT_Q6_K) return f16_bits_to_f32(lds_u16(s, row + 210u * (uint32_t)(p >> 3) + 208));
    if constexpr (QT == QT_Q8_0) return f16_bits_to_f32(lds_u16(s, row + 34u * (uint32_t)p));
}
template <int QT>
__device__ inline float block_dmin(const uint8_t* s, uint32_t row, int p) {
    if constexpr (QT == QT_Q4_K) return f16_bits_to_f32(lds_u16(s, row + 144u * (uint32_t)(p >> 3) + 2));
    return 0.0f;
}

// ---- integer dot of one item with its 32 activation bytes ---------------------
// Returns the item's exact integer contribution to its block sum; for Q4_K the
// min term is returned separately in `msum`.
template <int QT>
__device__ inline int item_dot(const Item& it, const uint32_t (&a)[8], const int16_t* bsum16, int p,
                               int& msum) {
    msum = 0;
    if constexpr (QT == QT_Q6_K) {
        int sa = 0, sb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) sa = __builtin_amdgcn_sdot4((int)it.v[i], (int)a[i], sa, false);
#pragma unroll
        for (int i = 4; i < 8; ++i) sb = __builtin_amdgcn_sdot4((int)it.v[i], (int)a[i], sb, false);
        // sum (q-32)*q8 = sum q*q8 - 32 * bsum over each 16-element half
        sa -= 32 * (int)bsum16[2 * p];
        sb -= 32 * (int)bsum16[2 * p + 1];
        return it.s0 * sa + it.s1 * sb;
    } else {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = __builtin_amdgcn_sdot4((int)it.v[i], (int)a[i], acc, false);
        if constexpr (QT == QT_Q4_K) {
            msum = it.s1 * ((int)bsum16[2 * p] + (int)bsum16[2 * p + 1]);
            return it.s0 * acc;
        }
        if constexpr (QT == QT_IQ3_S) return it.s0 * acc;
        return acc;   // Q8_0
    }
}

// ---- dequantised value of element l (0..31) of an item, in ggml's float order --
template <int QT>
__device__ inline float item_value(const Item& it, int l, float d, float dmin) {
    const int b = (int)((it.v[l >> 2] >> (8 * (l & 3))) & 0xFFu);
    if constexpr (QT == QT_IQ3_S) {
        // db = d * (1 + 2*scale); y = db * grid * sign
        const float db = __fmul_rn(d, (float)it.s0);
        return __fmul_rn(db, (float)(int8_t)b);
    }
    if constexpr (QT == QT_Q4_K) {
        // y = (d*sc) * q - (dmin*m)
        return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)it.s0), (float)b), __fmul_rn(dmin, (float)it.s1));
    }
    if constexpr (QT == QT_Q6_K) {
        // y = (d*sc) * (q - 32), sc of the 16-element half holding l
        const int sc = l < 16 ? it.s0 : it.s1;
        return __fmul_rn(__fmul_rn(d, (float)sc), (float)(b - 32));
    }
    if constexpr (QT == QT_Q8_0) return __fmul_rn((float)(int8_t)b, d);
}

}  // namespace sabah
