// Activation quantisation on the device: one fp32 row -> q8_0 or q8_K, in the
// ActLayout scratch form (quant_formats.h).  The integer values and scales are
// the ones ggml's CPU path feeds its vec_dot kernels:
//   q8_0 (quantize_row_q8_0_ref): per 32 elements d = amax/127 rounded to fp16,
//        q = roundf(x * (1/d)) (halves away from zero);
//   q8_K (quantize_row_q8_K_ref): per 256 elements the signed value of largest
//        magnitude (first on ties) gives iscale = -127/max, q = min(127, rint(iscale*x))
//        (nearest even), d = 1/iscale in fp32, bsums = sums of 16 consecutive q.
// The reference's own restatement of both steps is tools/rc4/opcheck.py:65-80.
//
// Work split: a wave64 owns one 256-element chunk at a time, four elements per
// lane, so every reduction is a lane shuffle inside the wave.
#pragma once
#include "quant_formats.h"

namespace sabah {

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ inline uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// Quantise one 256-element chunk (chunk index c of the row) held as float4 by
// the lanes of one wave.  Writes qs / d / bsum of that chunk into `act`.
__device__ inline void wave_quant_chunk_q8K(float4 v, int c, uint8_t* act, const ActLayout& L) {
    const int lane = threadIdx.x & 63;
    const float a0 = fabsf(v.x), a1 = fabsf(v.y), a2 = fabsf(v.z), a3 = fabsf(v.w);
    const float amax = wave_max(fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    // first element (in row order) whose magnitude equals amax
    int first = 0x7fffffff;
    float cand = 0.0f;
    if (a3 == amax) { first = 4 * lane + 3; cand = v.w; }
    if (a2 == amax) { first = 4 * lane + 2; cand = v.z; }
    if (a1 == amax) { first = 4 * lane + 1; cand = v.y; }
    if (a0 == amax) { first = 4 * lane + 0; cand = v.x; }
    const int fmin = wave_min_i(first);
    const float mx = __shfl(cand, (fmin == 0x7fffffff ? 0 : fmin) >> 2, 64);
    int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = __fdiv_rn(-127.0f, mx);
        q0 = min(127, (int)rintf(__fmul_rn(iscale, v.x)));
        q1 = min(127, (int)rintf(__fmul_rn(iscale, v.y)));
        q2 = min(127, (int)rintf(__fmul_rn(iscale, v.z)));
        q3 = min(127, (int)rintf(__fmul_rn(iscale, v.w)));
        d = __fdiv_rn(1.0f, iscale);
    }
    reinterpret_cast<uint32_t*>(act)[c * 64 + lane] = pack4_i8(q0, q1, q2, q3);
    // 16-element sums: four lanes per sum
    int s = q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(act + L.off_bsum)[c * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) reinterpret_cast<float*>(act + L.off_d)[c] = d;
}

// Same chunk shape for q8_0: eight 32-element blocks of eight lanes each.
__device__ inline void wave_quant_chunk_q8_0(float4 v, int c, uint8_t* act, const ActLayout& L) {
    const int lane = threadIdx.x & 63;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    const int q0 = (int)roundf(__fmul_rn(v.x, id));
    const int q1 = (int)roundf(__fmul_rn(v.y, id));
    const int q2 = (int)roundf(__fmul_rn(v.z, id));
    const int q3 = (int)roundf(__fmul_rn(v.w, id));
    reinterpret_cast<uint32_t*>(act)[c * 64 + lane] = pack4_i8(q0, q1, q2, q3);
    if ((lane & 7) == 0) {
        const float dh = __half2float(__float2half_rn(d));
        reinterpret_cast<float*>(act + L.off_d)[c * 8 + (lane >> 3)] = dh;
    }
}

// Load four consecutive floats of a row.  Rows handed over by the caller need
// not be 16-byte aligned (ggml views are 4-byte aligned), so fall back to
// scalar loads when they are not.
__device__ inline float4 load_f4(const float* p, bool aligned16) {
    if (aligned16) return *reinterpret_cast<const float4*>(p);
    return make_float4(p[0], p[1], p[2], p[3]);
}

// All threads of the workgroup: quantise the k floats at x into act.
// Requires k % 256 == 0 for q8_K and k % 32 == 0 for q8_0.
__device__ inline void wg_quantize_row(const float* __restrict__ x, int k, int at, uint8_t* act) {
    const ActLayout L(k, at);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const bool al = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const int nchunk = (k + 255) / 256;
    for (int c = wave; c < nchunk; c += nwave) {
        const int e = c * 256 + 4 * lane;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < k) v = load_f4(x + e, al);
        // lanes past k quantise zeros into the padding, which is never read
        if (at == QT_Q8_K) wave_quant_chunk_q8K(v, c, act, L);
        else wave_quant_chunk_q8_0(v, c, act, L);
    }
}

}  // namespace sabah
