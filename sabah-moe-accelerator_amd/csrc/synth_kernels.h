// Synthetic expert weights generated and quantised on the device.
//
// The benchmark bank (48 layers x 3 roles x 512 experts of IQ3_S, ~50 GB) is
// drawn from N(0, sigma) and encoded in HBM: one thread per quant block,
// normals from a counter-based hash (splitmix64 finaliser + Box-Muller) of the
// element index, so any block can be regenerated independently.  The
// encoders are simple valid ones (the same scheme as the oracle's); parity is
// judged on decoding identical bytes, which the CPU baseline reads back.
#pragma once
#include "quant_formats.h"

namespace sabah {

__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline float synth_normal(uint64_t seed, uint64_t idx) {
    const uint64_t h = mix64(mix64(seed) ^ (idx >> 1));
    const float u1 = (float)((h >> 40) + 1) * 5.9604645e-8f;           // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFull) * 5.9604645e-8f;  // [0, 1)
    const float r = sqrtf(-2.0f * __logf(u1));
    float s, c;
    __sincosf(6.2831853f * u2, &s, &c);
    return (idx & 1) ? r * s : r * c;
}

__device__ inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ inline void put_f16(uint8_t* p, float f) {
    const unsigned short h = __half_as_ushort(__float2half_rn(f));
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}
__device__ inline float get_f16(const uint8_t* p) {
    return __half2float(__ushort_as_half((unsigned short)(p[0] | (p[1] << 8))));
}

// element j of the block whose first element has global index e0
#define SYN(j) (sigma * synth_normal(seed, e0 + (uint64_t)(j)))

__device__ inline void enc_q8_0(uint8_t* y, uint64_t seed, uint64_t e0, float sigma) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(SYN(j)));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(y, d);
    for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(SYN(j) * id);
}

__device__ inline void enc_iq3_s(uint8_t* y, uint64_t seed, uint64_t e0, float sigma, const uint16_t* nearest) {
    for (int i = 0; i < 110; ++i) y[i] = 0;
    float am[8], A = 0.0f;
    for (int ib = 0; ib < 8; ++ib) {
        am[ib] = 0.0f;
        for (int j = 0; j < 32; ++j) am[ib] = fmaxf(am[ib], fabsf(SYN(32 * ib + j)));
        A = fmaxf(A, am[ib]);
    }
    if (A == 0.0f) return;
    put_f16(y, A / 465.0f);
    const float df = get_f16(y);
    if (df == 0.0f) { y[0] = y[1] = 0; return; }
    uint8_t *qs = y + 2, *qh = y + 66, *signs = y + 74, *scales = y + 106;
    for (int ib = 0; ib < 8; ++ib) {
        const int s = clampi((int)rintf((am[ib] / (15.0f * df) - 1.0f) * 0.5f), 0, 15);
        const float dl = df * (float)(2 * s + 1);
        scales[ib / 2] |= (uint8_t)(s << (4 * (ib & 1)));
        for (int g = 0; g < 8; ++g) {
            int key = 0;
            for (int j = 0; j < 4; ++j) {
                const float v = SYN(32 * ib + 4 * g + j);
                const int lv = clampi((int)rintf((fabsf(v) / dl - 1.0f) * 0.5f), 0, 7);
                key |= lv << (3 * j);
                if (v < 0.0f) signs[4 * ib + g / 2] |= (uint8_t)(1u << ((g & 1) * 4 + j));
            }
            const int gi = nearest[key];
            qs[8 * ib + g] = (uint8_t)(gi & 0xff);
            qh[ib] |= (uint8_t)((gi >> 8) << g);
        }
    }
}

__device__ inline void enc_q4_K(uint8_t* y, uint64_t seed, uint64_t e0, float sigma) {
    for (int i = 0; i < 144; ++i) y[i] = 0;
    float scl[8], mns[8], msc = 0.0f, mmn = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float lo = 0.0f, hi = 0.0f;
        for (int l = 0; l < 32; ++l) {
            const float v = SYN(32 * j + l);
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
        scl[j] = (hi - lo) / 15.0f;
        mns[j] = -lo;
        msc = fmaxf(msc, scl[j]);
        mmn = fmaxf(mmn, mns[j]);
    }
    put_f16(y, msc / 63.0f);
    put_f16(y + 2, mmn / 63.0f);
    const float df = get_f16(y), dmf = get_f16(y + 2);
    int sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = df > 0.0f ? clampi((int)rintf(scl[j] / df), 0, 63) : 0;
        mn[j] = dmf > 0.0f ? clampi((int)rintf(mns[j] / dmf), 0, 63) : 0;
    }
    uint8_t* p = y + 4;
    for (int j = 0; j < 4; ++j) {
        p[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        p[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        p[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    uint8_t* qs = y + 16;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) {
            int q[2];
            for (int hh = 0; hh < 2; ++hh) {
                const int j = 2 * c + hh;
                const float step = df * (float)sc[j], off = dmf * (float)mn[j];
                q[hh] = step > 0.0f ? clampi((int)rintf((SYN(64 * c + 32 * hh + l) + off) / step), 0, 15) : 0;
            }
            qs[32 * c + l] = (uint8_t)(q[0] | (q[1] << 4));
        }
}

__device__ inline void enc_q6_K(uint8_t* y, uint64_t seed, uint64_t e0, float sigma) {
    for (int i = 0; i < 210; ++i) y[i] = 0;
    float scl[16], ms = 0.0f;
    for (int j = 0; j < 16; ++j) {
        float am = 0.0f;
        for (int l = 0; l < 16; ++l) am = fmaxf(am, fabsf(SYN(16 * j + l)));
        scl[j] = am / 31.0f;
        ms = fmaxf(ms, scl[j]);
    }
    put_f16(y + 208, ms / 127.0f);
    const float df = get_f16(y + 208);
    int8_t* sc = reinterpret_cast<int8_t*>(y + 192);
    for (int j = 0; j < 16; ++j) sc[j] = (int8_t)(df > 0.0f ? clampi((int)rintf(scl[j] / df), -128, 127) : 0);
    uint8_t *ql = y, *qh = y + 128;
    for (int half = 0; half < 2; ++half)
        for (int l = 0; l < 32; ++l) {
            int u[4];
            for (int qq = 0; qq < 4; ++qq) {
                const int e = 128 * half + 32 * qq + l;
                const float step = df * (float)sc[e / 16];
                const int q = step != 0.0f ? clampi((int)rintf(SYN(e) / step), -32, 31) : 0;
                u[qq] = q + 32;
            }
            ql[64 * half + l] = (uint8_t)((u[0] & 0xF) | ((u[2] & 0xF) << 4));
            ql[64 * half + 32 + l] = (uint8_t)((u[1] & 0xF) | ((u[3] & 0xF) << 4));
            qh[32 * half + l] = (uint8_t)((u[0] >> 4) | ((u[1] >> 4) << 2) | ((u[2] >> 4) << 4) | ((u[3] >> 4) << 6));
        }
}
#undef SYN

// one thread per quant block; the workgroup's blocks are assembled in LDS and
// written out with coalesced stores.  grid = ceil(n_blocks / 256)
template <int QT>
__global__ __launch_bounds__(256) void k_synth(uint8_t* __restrict__ dst, long long n_blocks, uint64_t seed, float sigma,
                                               const uint16_t* __restrict__ nearest) {
    constexpr int QB = block_elems(QT), BB = block_bytes(QT);
    __shared__ __align__(16) uint8_t buf[256 * BB];
    const long long b0 = (long long)blockIdx.x * 256;
    const long long b = b0 + threadIdx.x;
    if (b < n_blocks) {
        uint8_t* y = buf + threadIdx.x * BB;
        const uint64_t e0 = (uint64_t)b * QB;
        if constexpr (QT == QT_IQ3_S) enc_iq3_s(y, seed, e0, sigma, nearest);
        if constexpr (QT == QT_Q4_K) enc_q4_K(y, seed, e0, sigma);
        if constexpr (QT == QT_Q6_K) enc_q6_K(y, seed, e0, sigma);
        if constexpr (QT == QT_Q8_0) enc_q8_0(y, seed, e0, sigma);
    }
    __syncthreads();
    const long long nvalid = (n_blocks - b0) < 256 ? (n_blocks - b0) : 256;
    const int nbytes = (int)nvalid * BB;
    uint8_t* out = dst + b0 * BB;
    if ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (nbytes & 15) == 0) {
        for (int q = threadIdx.x; q < nbytes / 16; q += 256)
            reinterpret_cast<uint4*>(out)[q] = reinterpret_cast<const uint4*>(buf)[q];
    } else {
        for (int q = threadIdx.x; q < nbytes; q += 256) out[q] = buf[q];
    }
}

}  // namespace sabah
