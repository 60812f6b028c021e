// Host-side decoding of the expert formats and quantisation of activations,
// for the library's CPU entry point (sabah_rt_host_dequant) and its sampled
// self-check of MUL_MAT_ID results (the reference's sb_host_dequant and
// sb_selfcheck, sabah_rt.cu:2233-2423 and 3435-3492).  Plain C++ on the host:
// no GPU, no initialisation.
//
// Values are produced with the same float steps as the device decoders
// (unit_decode.h unit_dequant) and ggml's dequantize_row_*, so
// sabah_rt_host_dequant agrees bit for bit with sabah_dequant.  The
// activation quantisers follow ggml's quantize_row_q8_{0,1,K}_ref, the
// integers the kernels' activations carry.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "quant_formats.h"

namespace sabah {
namespace host {

inline float half_to_float(const uint8_t* p) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return __half2float(__ushort_as_half(h));
}
inline uint16_t float_to_half_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }
inline float round_half(float f) { return __half2float(__float2half_rn(f)); }

inline uint32_t load_u32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}

// Q4_K / Q5_K sub-block j's 6-bit scale and min from the 12 packed bytes
inline void k_scale_min(const uint8_t* q, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

inline int8_t iq4_level(int i) { return (int8_t)((kIq4nlLevelWords[i >> 2] >> (8 * (i & 3))) & 0xFF); }

// k elements of type qt at x into y; false for an unsupported type or k
inline bool dequant_row(int qt, const uint8_t* x, float* y, int k) {
    if (!supported_weight_type(qt) || row_bytes(qt, k) == 0) return false;
    const int nb = k / block_elems(qt), bb = block_bytes(qt);
    for (int b = 0; b < nb; ++b, x += bb) {
        switch (qt) {
        case QT_Q8_0: {
            const float d = half_to_float(x);
            for (int j = 0; j < 32; ++j) *y++ = (float)(int8_t)x[2 + j] * d;
            break;
        }
        case QT_Q5_1: {
            const float d = half_to_float(x), m = half_to_float(x + 2);
            const uint32_t qh = load_u32(x + 4);
            for (int j = 0; j < 32; ++j) {
                const int nib = j < 16 ? (x[8 + j] & 0xF) : (x[8 + j - 16] >> 4);
                *y++ = (float)(nib | (int)(((qh >> j) & 1u) << 4)) * d + m;
            }
            break;
        }
        case QT_Q4_K:
        case QT_Q5_K: {
            const float d = half_to_float(x), dmin = half_to_float(x + 2);
            const uint8_t* qh = x + 16;
            const uint8_t* qs = x + (qt == QT_Q4_K ? 16 : 48);
            for (int j = 0; j < 8; ++j) {
                int sc, mn;
                k_scale_min(x + 4, j, sc, mn);
                const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                for (int l = 0; l < 32; ++l) {
                    int q = (qs[32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF;
                    if (qt == QT_Q5_K) q += ((qh[l] >> j) & 1) * 16;
                    *y++ = d1 * (float)q - m1;
                }
            }
            break;
        }
        case QT_Q6_K: {
            const uint8_t *ql = x, *qh = x + 128;
            const int8_t* sc = reinterpret_cast<const int8_t*>(x + 192);
            const float d = half_to_float(x + 208);
            for (int e = 0; e < 256; ++e) {
                const int h = e >> 7, r = e & 127, quarter = r >> 5, l = r & 31;
                const int lo = (ql[64 * h + 32 * (quarter & 1) + l] >> (4 * (quarter >> 1))) & 0xF;
                const int hi = (qh[32 * h + l] >> (2 * quarter)) & 3;
                *y++ = d * (float)sc[8 * h + 2 * quarter + (l >> 4)] * (float)((lo | (hi << 4)) - 32);
            }
            break;
        }
        case QT_IQ3_S: {
            static const Iq3sGrid grid = make_iq3s_grid();
            const float d = half_to_float(x);
            const uint8_t *qs = x + 2, *qh = x + 66, *signs = x + 74, *scales = x + 106;
            for (int ib = 0; ib < 8; ++ib) {
                const float db = d * (float)(2 * ((scales[ib >> 1] >> (4 * (ib & 1))) & 0xF) + 1);
                for (int g = 0; g < 8; ++g) {
                    const uint32_t e = grid.e[qs[8 * ib + g] | (((qh[ib] >> g) & 1) << 8)];
                    for (int j = 0; j < 4; ++j) {
                        const int mag = (int)((e >> (8 * j)) & 0xFF);
                        const bool neg = (signs[4 * ib + (g >> 1)] >> (4 * (g & 1) + j)) & 1;
                        *y++ = db * (float)(neg ? -mag : mag);
                    }
                }
            }
            break;
        }
        case QT_IQ3_XXS: {
            const float d = half_to_float(x);
            const uint8_t *qs = x + 2, *ss = x + 66;
            for (int ib = 0; ib < 8; ++ib) {
                const uint32_t aux = load_u32(ss + 4 * ib);
                const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
                for (int l = 0; l < 4; ++l) {
                    uint32_t sg = (aux >> (7 * l)) & 127u;
                    sg |= (uint32_t)(__builtin_popcount(sg) & 1) << 7;
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t e = kIq3xxsGridWords[qs[8 * ib + 2 * l + h]];
                        for (int j = 0; j < 4; ++j) {
                            const int mag = (int)((e >> (8 * j)) & 0xFF);
                            *y++ = db * (float)(((sg >> (4 * h + j)) & 1) ? -mag : mag);
                        }
                    }
                }
            }
            break;
        }
        case QT_IQ2_S: {
            const float d = half_to_float(x);
            const uint8_t *qs = x + 2, *signs = x + 34, *qh = x + 66, *sc = x + 74;
            for (int ib = 0; ib < 8; ++ib) {
                const float db0 = d * (0.5f + (float)(sc[ib] & 0xF)) * 0.25f;
                const float db1 = d * (0.5f + (float)(sc[ib] >> 4)) * 0.25f;
                for (int l = 0; l < 4; ++l) {
                    const int gi = qs[4 * ib + l] | (((qh[ib] >> (2 * l)) & 3) << 8);
                    const uint64_t e = (uint64_t)kIq2sGridWords[2 * gi] | ((uint64_t)kIq2sGridWords[2 * gi + 1] << 32);
                    for (int j = 0; j < 8; ++j) {
                        const int mag = (int)((e >> (8 * j)) & 0xFF);
                        *y++ = (l < 2 ? db0 : db1) * (float)(((signs[4 * ib + l] >> j) & 1) ? -mag : mag);
                    }
                }
            }
            break;
        }
        case QT_IQ4_NL: {
            const float d = half_to_float(x);
            for (int j = 0; j < 32; ++j) *y++ = d * (float)iq4_level(j < 16 ? x[2 + j] & 0xF : x[2 + j - 16] >> 4);
            break;
        }
        case QT_IQ4_XS: {
            const float d = half_to_float(x);
            const int sh = x[2] | (x[3] << 8);
            const uint8_t *sl = x + 4, *qs = x + 8;
            for (int ib = 0; ib < 8; ++ib) {
                const int ls = ((sl[ib >> 1] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                for (int j = 0; j < 32; ++j)
                    *y++ = dl * (float)iq4_level(j < 16 ? qs[16 * ib + j] & 0xF : qs[16 * ib + j - 16] >> 4);
            }
            break;
        }
        case QT_Q2_0: {
            const float d = half_to_float(x);
            for (int j = 0; j < 64; ++j) *y++ = (float)(((x[2 + (j >> 2)] >> (2 * (j & 3))) & 3) - 1) * d;
            break;
        }
        default:
            return false;
        }
    }
    return true;
}

// The activation row the kernels dot a weight row of type qt with, as
// doubles (q * d), plus, for q8_1 (Q5_1 weights), each 32-block's stored s.
struct ActRow {
    std::vector<double> v;      // k values q * d
    std::vector<double> s;      // q8_1 only: per 32-block fp16 s = d * sum(q)
};

inline void quantize_act(int qt, const float* x, int k, ActRow& a) {
    const int at = act_type(qt);
    a.v.assign(k, 0.0);
    a.s.clear();
    if (at == QT_Q8_K) {
        for (int b = 0; b < k / 256; ++b) {
            const float* xb = x + 256 * b;
            float amax = 0.0f, mx = 0.0f;
            for (int j = 0; j < 256; ++j)
                if (std::fabs(xb[j]) > amax) amax = std::fabs(xb[j]), mx = xb[j];
            if (amax == 0.0f) continue;
            const float iscale = -127.0f / mx;
            const float d = 1.0f / iscale;
            for (int j = 0; j < 256; ++j) {
                const int q = std::min(127, (int)std::nearbyint(iscale * xb[j]));
                a.v[256 * b + j] = (double)q * (double)d;
            }
        }
        return;
    }
    for (int b = 0; b < k / 32; ++b) {              // q8_0, q8_1
        const float* xb = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const double dh = (double)round_half(d);
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            const int q = (int)std::round(xb[j] * id);
            sum += q;
            a.v[32 * b + j] = (double)q * dh;
        }
        if (at == QT_Q8_1) a.s.push_back((double)round_half((float)sum * d));
    }
}

// float64 value of one output: weight row (decoded into w) . activation row;
// Q5_1 takes its min term from the activation's s, as ggml's dot does
inline double ref_dot(int qt, const uint8_t* wrow, const float* w, const ActRow& a, int k) {
    double acc = 0.0;
    if (qt == QT_Q5_1) {
        for (int b = 0; b < k / 32; ++b) {
            const double m = (double)half_to_float(wrow + 24 * b + 2);
            for (int j = 0; j < 32; ++j) acc += ((double)w[32 * b + j] - m) * a.v[32 * b + j];
            acc += m * a.s[b];
        }
        return acc;
    }
    for (int c = 0; c < k; ++c) acc += (double)w[c] * a.v[c];
    return acc;
}

}  // namespace host
}  // namespace sabah
