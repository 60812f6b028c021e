// Activation quantisation on the device: fp32 rows -> q8_0, q8_1 or q8_K, in the
// ActLayout scratch form (quant_formats.h).  The integer values and scales are
// the ones ggml's CPU path feeds its vec_dot kernels:
//   q8_0 (quantize_row_q8_0_ref): per 32 elements d = amax/127 rounded to fp16,
//        q = roundf(x * (1/d)) (halves away from zero);
//   q8_1 (quantize_row_q8_1_ref): q8_0's d and q, plus s = sum(q) * d rounded to fp16;
//   q8_K (quantize_row_q8_K_ref): per 256 elements the signed value of largest
//        magnitude (first on ties) gives iscale = -127/max, q = min(127, rint(iscale*x))
//        (nearest even), d = 1/iscale in fp32, bsums = sums of 16 consecutive q.
// The reference's own restatement of both steps is tools/rc4/opcheck.py:65-80.
//
// Work split: sixteen lanes (one DPP row) own one 256-element chunk, sixteen
// consecutive elements per lane, so a wave quantises four chunks at once,
// every reduction is four DPP steps inside the row, and each lane's sixteen
// values are exactly one q8_K bsum.
#pragma once
#include "quant_formats.h"

namespace sabah {

// floor(a / b) for 0 <= a < 2^21, given r = rcp(b) (v_rcp_f32, 1 ulp): the
// product's relative error stays below 2^-22, so its absolute error is below
// (a + 0.5) / b * 2^-22 < 0.5 / b, while (a + 0.5) / b is at least 0.5 / b
// away from an integer
__device__ inline int div_small(int a, float r) { return (int)(((float)a + 0.5f) * r); }
// the same for wave-uniform operands, returned as a scalar
__device__ inline int div_small_u(int a, float r) { return __builtin_amdgcn_readfirstlane(div_small(a, r)); }
__device__ inline int div_small_u(int a, int b) { return div_small_u(a, __builtin_amdgcn_rcpf((float)b)); }


template <int CTRL>
__device__ inline uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8-lane half-row
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16-lane row

__device__ inline float row16_max(float v) {
    v = fmaxf(v, __uint_as_float(dpp<kDppXor1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp<kDppXor2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp<kDppMirror>(__float_as_uint(v))));
    return v;
}
__device__ inline uint32_t row16_min(uint32_t v) {
    v = min(v, dpp<kDppXor1>(v));
    v = min(v, dpp<kDppXor2>(v));
    v = min(v, dpp<kDppHalfMirror>(v));
    v = min(v, dpp<kDppMirror>(v));
    return v;
}

__device__ inline int sdot4_i8(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

__device__ inline uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// sixteen consecutive floats of one lane
struct Act16 {
    float v[16];
};

__device__ inline float row16_min(float v) {
    v = fminf(v, __uint_as_float(dpp<kDppXor1>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(dpp<kDppXor2>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(dpp<kDppHalfMirror>(__float_as_uint(v))));
    v = fminf(v, __uint_as_float(dpp<kDppMirror>(__float_as_uint(v))));
    return v;
}

// ggml's nearest_int: v + 1.5 * 2^23 rounds v to an integer (nearest, ties
// to even) for |v| < 2^22, leaving it in the low mantissa bits; the float's
// bits are then 0x4B400000 + nearest_int(v), so the low byte is the int8.
constexpr float kRoundMagic = 12582912.0f;
constexpr uint32_t kRoundMagicBits = 0x4B400000u;

// bytes 0 of a, b, c, d -> one dword (a in byte 0)
__device__ inline uint32_t low_bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);   // [a.0, b.0, 0, 0]
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x04000C0Cu);   // [0, 0, c.0, d.0]
    return ab | cd;
}

// Quantise the chunk held by one 16-lane row (lane l holds elements 16l..16l+15)
// into act (the row's ActLayout block), chunk index c.
//
// The scale comes from the first element of largest magnitude, with its sign.
// Unless both +amax and -amax occur in the chunk, that sign is the sign of
// whichever of the chunk's maximum and minimum reaches amax; only a chunk
// holding both looks for the first one by index.  |iscale * x| <= 127 (1 + 2^-22)
// rounds to at most 127, so ggml's clamp at 127 never applies.
// mfma_order: the chunk's 256 bytes in the grouped kernels' operand order, in
// which the element k = 32 s + 8 q + i (sub-block s, quarter q, i < 8) sits
// at byte 64 (s / 2) + 16 q + 8 (s % 2) + i, so one 16-byte load gives an
// MFMA lane its eight elements of two sub-blocks (bsums and d unchanged).
__device__ inline void row16_quant_q8K(const Act16& a, int c, uint8_t* act, const ActLayout& L, bool mfma_order = false) {
    const uint32_t l = threadIdx.x & 15u;
    float mx_l = a.v[0], mn_l = a.v[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) {
        mx_l = fmaxf(mx_l, a.v[j]);
        mn_l = fminf(mn_l, a.v[j]);
    }
    const float rmax = row16_max(mx_l), rmin = row16_min(mn_l);
    const float amax = fmaxf(rmax, -rmin);
    float mx = rmax == amax ? amax : -amax;
    if (rmax == amax && rmin == -amax && amax != 0.0f) {     // both signs reach amax: the first one decides
        uint32_t key = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 15; j >= 0; --j)
            if (fabsf(a.v[j]) == amax) key = ((16u * l + (uint32_t)j) << 1) | (__float_as_uint(a.v[j]) >> 31);
        key = row16_min(key);
        mx = (key & 1u) ? -amax : amax;
    }
    uint32_t b[16];
    float d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
        for (int j = 0; j < 16; ++j) b[j] = __float_as_uint(__fadd_rn(__fmul_rn(iscale, a.v[j]), kRoundMagic));
        d = __fdiv_rn(1.0f, iscale);
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) b[j] = kRoundMagicBits;
    }
    uint4 packed;
    packed.x = low_bytes4(b[0], b[1], b[2], b[3]);
    packed.y = low_bytes4(b[4], b[5], b[6], b[7]);
    packed.z = low_bytes4(b[8], b[9], b[10], b[11]);
    packed.w = low_bytes4(b[12], b[13], b[14], b[15]);
    if (mfma_order) {
        // elements 16 l .. 16 l + 7 and 16 l + 8 .. + 15: quarters 2 (l & 1) and 2 (l & 1) + 1 of sub-block l / 2
        uint8_t* o = act + c * kActChunkStride + 64 * (l >> 2) + 32 * (l & 1u) + 8 * ((l >> 1) & 1u);
        *reinterpret_cast<uint2*>(o) = make_uint2(packed.x, packed.y);
        *reinterpret_cast<uint2*>(o + 16) = make_uint2(packed.z, packed.w);
    } else {
        reinterpret_cast<uint4*>(act + c * kActChunkStride)[l] = packed;
    }
    // bsum = sum of the sixteen int8 values
    int s = 0;
    s = sdot4_i8(packed.x, 0x01010101u, s);
    s = sdot4_i8(packed.y, 0x01010101u, s);
    s = sdot4_i8(packed.z, 0x01010101u, s);
    s = sdot4_i8(packed.w, 0x01010101u, s);
    reinterpret_cast<int16_t*>(act + L.off_bsum)[c * 16 + l] = (int16_t)s;
    if (l == 0) reinterpret_cast<float*>(act + L.off_d)[c] = d;
}

// q8_0: the 32-element block b of the chunk is lanes 2b and 2b+1.  q8_1
// (with_sum) also stores s = fp16(sum(q) * d), d the fp32 scale before its
// fp16 rounding (quantize_row_q8_1_ref), in the layout's s area.
__device__ inline void row16_quant_q8_0(const Act16& a, int c, uint8_t* act, const ActLayout& L,
                                        bool with_sum = false) {
    const uint32_t l = threadIdx.x & 15u;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(a.v[j]));
    amax = fmaxf(amax, __uint_as_float(dpp<kDppXor1>(__float_as_uint(amax))));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    int q[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] = (int)roundf(__fmul_rn(a.v[j], id));
    uint4 packed;
    packed.x = pack4_i8(q[0], q[1], q[2], q[3]);
    packed.y = pack4_i8(q[4], q[5], q[6], q[7]);
    packed.z = pack4_i8(q[8], q[9], q[10], q[11]);
    packed.w = pack4_i8(q[12], q[13], q[14], q[15]);
    reinterpret_cast<uint4*>(act + c * kActChunkStride)[l] = packed;
    if ((l & 1u) == 0) reinterpret_cast<float*>(act + L.off_d)[c * 8 + (l >> 1)] = __half2float(__float2half_rn(d));
    if (with_sum) {
        int s = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) s += q[j];
        s += (int)dpp<kDppXor1>((uint32_t)s);            // the block's other sixteen
        // the fp32 product is rounded before its fp16 rounding: the empty asm
        // keeps the compiler from selecting one mixed-precision multiply that
        // rounds the exact product to fp16 once (a tie of the fp32 product
        // then rounds differently)
        float sd = __fmul_rn((float)s, d);
        asm volatile("" : "+v"(sd));
        if ((l & 1u) == 0)
            reinterpret_cast<float*>(act + L.off_bsum)[c * 8 + (l >> 1)] = __half2float(__float2half_rn(sd));
    }
}

// Load sixteen consecutive floats: elements e..e+15 of a row of k (k is a
// multiple of 16, so a lane's sixteen are all in the row or all past it).
// Every lane issues the same loads (a lane past the row re-reads the row's
// first sixteen, which act_quantize replaces by zeros), so the number of
// loads in flight is static.  `vec` (uniform: row pointers 16-byte aligned)
// selects four 16-byte loads; rows need only be 4-byte aligned.
__device__ inline void load16(const float* row, int e, int k, bool vec, Act16& a) {
    const float* p = row + (e < k ? e : 0);
    if (vec) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 f = reinterpret_cast<const float4*>(p)[i];
            a.v[4 * i] = f.x; a.v[4 * i + 1] = f.y; a.v[4 * i + 2] = f.z; a.v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) a.v[j] = p[j];
    }
}

// An activation batch: n_rows rows of k floats, row_stride floats apart,
// quantised into ActLayout blocks act_stride bytes apart.  Chunk-row q (row
// q / nch, chunk q % nch) belongs to row-slot q % nslots (a row-slot is one
// 16-lane DPP row of the workgroup) in round q / nslots.
struct ActBatch {
    const float* x;
    size_t row_stride;
    int n_rows, k, at;
    uint8_t* act;
    int act_stride;
};

// Split form: the loads (act_prefetch) are issued early and the quantisation
// (act_quantize) runs later, so the caller can issue its own long-latency
// loads in between.  Rounds past ROUNDS fall back to load-then-quantise.
template <int ROUNDS>
struct ActRegs {
    Act16 a[ROUNDS];
};

// The batch is handled by threads w0 .. NT-1 (whole 16-lane rows) of a
// workgroup of NT threads (a constant, so no kernel reads its launch size).
__device__ inline bool act_vec(const ActBatch& B) {
    return (reinterpret_cast<uintptr_t>(B.x) & 15) == 0 && (B.row_stride & 3) == 0;
}

// every lane loads in every round (slots past the batch re-load its last
// chunk-row and skip the quantisation)
template <int ROUNDS, int NT>
__device__ inline void act_prefetch(const ActBatch& B, ActRegs<ROUNDS>& R, int w0 = 0) {
    const int slot = ((int)threadIdx.x - w0) >> 4, nslots = (NT - w0) >> 4, l = threadIdx.x & 15;
    const int nch = (B.k + 255) / 256, nq = B.n_rows * nch;
    const float rcp_nch = __builtin_amdgcn_rcpf((float)nch);
    const bool vec = act_vec(B);
#pragma unroll
    for (int i = 0; i < ROUNDS; ++i) {
        const int q = min(slot + nslots * i, nq - 1);
        const int r = div_small(q, rcp_nch), c = q - r * nch;
        load16(B.x + (size_t)r * B.row_stride, c * 256 + 16 * l, B.k, vec, R.a[i]);
    }
}

__device__ inline void quant_chunk(const ActBatch& B, const Act16& a_in, int q, bool mfma_order = false) {
    const int nch = (B.k + 255) / 256;
    const int r = div_small(q, __builtin_amdgcn_rcpf((float)nch)), c = q - r * nch;
    const ActLayout L(B.k, B.at);
    const bool in = c * 256 + 16 * (int)(threadIdx.x & 15u) < B.k;
    Act16 a;
#pragma unroll
    for (int j = 0; j < 16; ++j) a.v[j] = in ? a_in.v[j] : 0.0f;
    if (B.at == QT_Q8_K) row16_quant_q8K(a, c, B.act + r * B.act_stride, L, mfma_order);
    else row16_quant_q8_0(a, c, B.act + r * B.act_stride, L, B.at == QT_Q8_1);
}

template <int ROUNDS, int NT>
__device__ inline void act_quantize(const ActBatch& B, const ActRegs<ROUNDS>& R, int w0 = 0) {
    const int slot = ((int)threadIdx.x - w0) >> 4, nslots = (NT - w0) >> 4, l = threadIdx.x & 15;
    const int nch = (B.k + 255) / 256, nq = B.n_rows * nch;
#pragma unroll
    for (int i = 0; i < ROUNDS; ++i) {
        const int q = slot + nslots * i;
        if (q < nq) quant_chunk(B, R.a[i], q);
    }
    const bool vec = act_vec(B);
    const float rcp_nch = __builtin_amdgcn_rcpf((float)nch);
    for (int q = slot + nslots * ROUNDS; q < nq; q += nslots) {
        const int r = div_small(q, rcp_nch), c = q - r * nch;
        Act16 a;
        load16(B.x + (size_t)r * B.row_stride, c * 256 + 16 * l, B.k, vec, a);
        quant_chunk(B, a, q);
    }
}

// All threads of a 256-thread workgroup: quantise one row of k floats at x into act.
__device__ inline void wg_quantize_row(const float* __restrict__ x, int k, int at, uint8_t* act) {
    const ActBatch B{x, 0, 1, k, at, act, 0};
    ActRegs<1> R;
    act_prefetch<1, 256>(B, R);
    act_quantize<1, 256>(B, R);
}

}  // namespace sabah
