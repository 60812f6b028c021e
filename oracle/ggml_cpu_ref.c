/*
 * ORACLE - test infrastructure only (see ggml_cpu_ref.h).
 *
 * Restatement of ggml's portable CPU path for MUL_MAT_ID on Q8_0 / Q5_1 /
 * Q4_K / Q5_K / Q6_K / IQ3_S (and the other IQ) expert weights.  ggml (llama.cpp @ 96ffdc41) is a third-party
 * dependency that the reference does not vendor; the algorithm followed here
 * is its published generic C form:
 *   quantize_row_q8_0_ref, quantize_row_q8_1_ref, quantize_row_q8_K_ref
 *                                                        (activation quantisers)
 *   dequantize_row_{q8_0,q4_K,q6_K,iq3_s}                (format readers)
 *   ggml_vec_dot_{q8_0_q8_0,q5_1_q8_1,q4_K_q8_K,q5_K_q8_K,q6_K_q8_K,iq3_s_q8_K}_generic
 *   ggml_compute_forward_mul_mat_id                      (slot i reads row i % ne11)
 * anchored on the reference's own readers of the same formats
 * (sabah_rt.cu:2233-2423; gguf-py quants.py:412-435, 509-556, 586-606,
 * 1091-1159) and its description of the activation step (tools/rc4/opcheck.py:65-83).
 *
 * Build with -ffp-contract=off: every float operation below is meant to round
 * on its own, as in the C source it restates.
 */
#include "ggml_cpu_ref.h"
#include "iq3s_grid_u32.h"
#include "iq_tables_u32.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_block_elems(int qt) {
    switch (qt) {
    case ORC_Q8_0: case ORC_Q8_1: case ORC_Q5_1: case ORC_IQ4_NL: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: case ORC_IQ3_S: case ORC_IQ3_XXS: case ORC_IQ4_XS:
    case ORC_IQ2_S: return 256;
    case ORC_Q2_0: return 64;
    }
    return 0;
}

int orc_block_bytes(int qt) {
    switch (qt) {
    case ORC_Q8_0: return 34;    /* fp16 d + 32 x int8                       */
    case ORC_Q8_1: return 36;    /* fp16 d, fp16 s = d * sum(q), 32 x int8   */
    case ORC_Q5_1: return 24;    /* fp16 d, fp16 m, u32 qh, 16 B nibbles     */
    case ORC_Q5_K: return 176;   /* d, dmin, 12 B scales/mins, qh[32], qs[128] */
    case ORC_Q4_K: return 144;   /* d, dmin, 12 B scales/mins, 128 B nibbles */
    case ORC_Q6_K: return 210;   /* ql[128], qh[64], int8 sc[16], fp16 d      */
    case ORC_Q8_K: return 292;   /* float d, int8 qs[256], int16 bsums[16]    */
    case ORC_IQ3_S: return 110;  /* d, qs[64], qh[8], signs[32], scales[4]    */
    case ORC_IQ3_XXS: return 98; /* d, qs[64] grid indices, 8 x u32 scale/signs */
    case ORC_IQ2_S: return 82;   /* d, qs[32], signs[32], qh[8], scales[8]       */
    case ORC_IQ4_NL: return 18;  /* d, 16 B nibbles                          */
    case ORC_IQ4_XS: return 136; /* d, scales_h u16, scales_l[4], qs[128]     */
    case ORC_Q2_0: return 18;    /* d, 16 B of 2-bit codes (sabah_rt.cu:2166)  */
    }
    return 0;
}

size_t orc_row_bytes(int qt, int n) {
    const int be = orc_block_elems(qt);
    if (be == 0 || n % be) return 0;
    return (size_t)(n / be) * (size_t)orc_block_bytes(qt);
}

int orc_vec_dot_type(int qt) {
    switch (qt) {
    case ORC_Q8_0: case ORC_IQ4_NL: case ORC_Q2_0: return ORC_Q8_0;
    case ORC_Q5_1: return ORC_Q8_1;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_IQ3_S: case ORC_IQ3_XXS: case ORC_IQ4_XS: case ORC_IQ2_S:
        return ORC_Q8_K;
    }
    return -1;
}

size_t orc_act_row_bytes(int qt, int k) {
    const int vt = orc_vec_dot_type(qt);
    return vt < 0 ? 0 : orc_row_bytes(vt, k);
}

/* ------------------------------------------------------------------------ */
/* binary16                                                                  */
/* ------------------------------------------------------------------------ */
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                       /* subnormal: m * 2^-24 */
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                         /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds to inf */
    const uint32_t e = ax >> 23;
    if (e < 113) {                                   /* result is subnormal or zero */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t s = 126 - e;                  /* value / 2^-24 = m >> s     */
        if (e == 0 || s > 24) return sign;           /* < half a unit: rounds to 0 */
        uint32_t q = m >> s;
        const uint32_t rem = m & ((1u << s) - 1u), half = 1u << (s - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((e - 112) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;     /* may carry into exponent */
    return (uint16_t)(sign | h);
}

static inline float ld_f16(const uint8_t *p) { return orc_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }
static inline void st_f16(uint8_t *p, float f) { const uint16_t h = orc_fp32_to_fp16(f); p[0] = (uint8_t)h; p[1] = (uint8_t)(h >> 8); }

/* ------------------------------------------------------------------------ */
/* activation quantisers                                                     */
/* ------------------------------------------------------------------------ */

/* quantize_row_q8_0_ref: d = amax/127 (stored fp16), q = roundf(x * (1/d)),
 * halves away from zero (quants.py:412-427 restates the same steps and calls
 * them bit-exact with ggml-quants.c). */
void orc_quantize_q8_0(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 32; ++b, x += 32, y += 34) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = fabsf(x[j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_f16(y, d);
        for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
    }
}

/* quantize_row_q8_1_ref: the q8_0 steps (d = amax/127 stored fp16, q =
 * roundf(x * (1/d)) with the fp32 d), plus s = fp16((float)sum(q) * d), the
 * fp32 d again (ggml-quants.c; the vec_dot_type of Q5_1, sabah_rt.cu's Q5_1
 * readers at 2241-2252 and 2522-2541 take the same block). */
void orc_quantize_q8_1(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 32; ++b, x += 32, y += 36) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = fabsf(x[j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_f16(y, d);
        int sum = 0;
        for (int j = 0; j < 32; ++j) {
            const int q = (int)roundf(x[j] * id);
            y[4 + j] = (uint8_t)(int8_t)q;
            sum += q;
        }
        st_f16(y + 2, (float)sum * d);
    }
}

/* quantize_row_q8_K_ref: the signed value of largest magnitude (first one on
 * ties) sets iscale = -127/max; q = min(127, nearest-even(iscale*x)); d = 1/iscale
 * kept in fp32; bsums[j] = sum of q over elements 16j..16j+15.  opcheck.py:73-80
 * restates the same q and d. */
void orc_quantize_q8_K(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 256; ++b, x += 256, y += 292) {
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        int8_t *qs = (int8_t *)(y + 4);
        int16_t bs[16];
        if (amax == 0.0f) {
            memset(y, 0, 292);
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < 256; ++j) {
            const int v = (int)rintf(iscale * x[j]);
            qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += qs[16 * j + i];
            bs[j] = (int16_t)s;
        }
        memcpy(y + 260, bs, sizeof(bs));
        const float d = 1.0f / iscale;
        memcpy(y, &d, 4);
    }
}

int orc_quantize_act(int qt, const float *x, uint8_t *y, int k) {
    const int vt = orc_vec_dot_type(qt);
    if (vt < 0 || k % orc_block_elems(vt)) return -1;
    if (vt == ORC_Q8_0) orc_quantize_q8_0(x, y, k);
    else if (vt == ORC_Q8_1) orc_quantize_q8_1(x, y, k);
    else orc_quantize_q8_K(x, y, k);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* decoders (dequantize_row_*)                                               */
/* ------------------------------------------------------------------------ */

/* get_scale_min_k4: sub-block j's 6-bit scale and min from the 12 packed bytes
 * (sabah_rt.cu:2210-2218 host form, quants.py:513-536 unpacking diagram). */
static inline void scale_min_k4(int j, const uint8_t *q, int *sc, int *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

int orc_dequantize_row(int qt, const uint8_t *x, float *y, int k) {
    if (orc_row_bytes(qt, k) == 0) return -1;
    switch (qt) {
    case ORC_Q8_0:
        for (int b = 0; b < k / 32; ++b, x += 34) {
            const float d = ld_f16(x);
            for (int j = 0; j < 32; ++j) *y++ = (float)(int8_t)x[2 + j] * d;
        }
        return 0;
    case ORC_Q4_K:
        for (int b = 0; b < k / 256; ++b, x += 144) {
            const float d = ld_f16(x), dmin = ld_f16(x + 2);
            const uint8_t *sc = x + 4, *q = x + 16;
            for (int c = 0; c < 4; ++c, q += 32) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * c, sc, &s0, &m0);
                scale_min_k4(2 * c + 1, sc, &s1, &m1);
                const float d1 = d * (float)s0, n1 = dmin * (float)m0;
                const float d2 = d * (float)s1, n2 = dmin * (float)m1;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (float)(q[l] & 0xF) - n1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (float)(q[l] >> 4) - n2;
            }
        }
        return 0;
    case ORC_Q5_1:
        /* element j (j < 16) = (qs[j] & 15) | bit j of qh << 4, element j + 16 =
         * (qs[j] >> 4) | bit j + 16 of qh << 4; value = d * q + m
         * (sabah_rt.cu:2241-2252, quants.py:390-409) */
        for (int b = 0; b < k / 32; ++b, x += 24, y += 32) {
            const float d = ld_f16(x), m = ld_f16(x + 2);
            const uint32_t qh = (uint32_t)x[4] | ((uint32_t)x[5] << 8) | ((uint32_t)x[6] << 16) | ((uint32_t)x[7] << 24);
            const uint8_t *qs = x + 8;
            for (int j = 0; j < 16; ++j) {
                const int q0 = (qs[j] & 0xF) | (int)(((qh >> j) & 1u) << 4);
                const int q1 = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
                y[j] = (float)q0 * d + m;
                y[j + 16] = (float)q1 * d + m;
            }
        }
        return 0;
    case ORC_Q5_K:
        /* sub-block j, element l: nibble (low for even j) of qs[32 (j / 2) + l]
         * plus 16 when bit j of qh[l] is set; value = d * sc_j * q - dmin * m_j
         * (sabah_rt.cu:2271-2290, quants.py:559-583) */
        for (int b = 0; b < k / 256; ++b, x += 176) {
            const float d = ld_f16(x), dmin = ld_f16(x + 2);
            const uint8_t *sc = x + 4, *qh = x + 16, *q = x + 48;
            for (int c = 0; c < 4; ++c, q += 32) {
                int s0, m0, s1, m1;
                scale_min_k4(2 * c, sc, &s0, &m0);
                scale_min_k4(2 * c + 1, sc, &s1, &m1);
                const float d1 = d * (float)s0, n1 = dmin * (float)m0;
                const float d2 = d * (float)s1, n2 = dmin * (float)m1;
                for (int l = 0; l < 32; ++l) *y++ = d1 * (float)((q[l] & 0xF) + ((qh[l] >> (2 * c)) & 1) * 16) - n1;
                for (int l = 0; l < 32; ++l) *y++ = d2 * (float)((q[l] >> 4) + ((qh[l] >> (2 * c + 1)) & 1) * 16) - n2;
            }
        }
        return 0;
    case ORC_Q6_K:
        for (int b = 0; b < k / 256; ++b, x += 210) {
            const uint8_t *ql = x, *qh = x + 128;
            const int8_t *sc = (const int8_t *)(x + 192);
            const float d = ld_f16(x + 208);
            for (int half = 0; half < 2; ++half, y += 128, ql += 64, qh += 32, sc += 8) {
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float)sc[is] * (float)q1;
                    y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
        return 0;
    case ORC_IQ3_S:
        for (int b = 0; b < k / 256; ++b, x += 110) {
            const float d = ld_f16(x);
            const uint8_t *qs = x + 2, *qh = x + 66, *signs = x + 74, *scales = x + 106;
            for (int ib = 0; ib < 8; ++ib) {
                const float db = d * (float)(1 + 2 * ((scales[ib / 2] >> (4 * (ib & 1))) & 0xF));
                for (int g = 0; g < 8; ++g) {
                    const uint32_t gi = (uint32_t)qs[8 * ib + g] | (((uint32_t)(qh[ib] >> g) & 1u) << 8);
                    const uint32_t grid = orc_iq3s_grid[gi];
                    const uint8_t sg = signs[4 * ib + g / 2];
                    for (int j = 0; j < 4; ++j) {
                        const int bit = (g & 1) * 4 + j;
                        *y++ = db * (float)((grid >> (8 * j)) & 0xFF) * ((sg >> bit) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
        }
        return 0;
    case ORC_IQ2_S:     /* sabah_rt.cu:2293-2318; quants.py:935-1037 */
        /* element 32 ib + 8 l + j = db(l) * grid[qs[4 ib + l] | qh bits 2l..2l+1 << 8][j]
         * * (-1 if bit j of signs[4 ib + l]); db = d * (0.5 + nibble) * 0.25, the low
         * nibble of scales[ib] for l < 2, the high one for l >= 2 */
        for (int b = 0; b < k / 256; ++b, x += 82) {
            const float d = ld_f16(x);
            const uint8_t *qs = x + 2, *signs = x + 34, *qh = x + 66, *sc = x + 74;
            for (int ib = 0; ib < 8; ++ib) {
                const float db0 = d * (0.5f + (float)(sc[ib] & 0xF)) * 0.25f;
                const float db1 = d * (0.5f + (float)(sc[ib] >> 4)) * 0.25f;
                for (int l = 0; l < 4; ++l) {
                    const float dl = l < 2 ? db0 : db1;
                    const uint64_t g = orc_iq2s_grid[qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300)];
                    const uint8_t sg = signs[4 * ib + l];
                    for (int j = 0; j < 8; ++j)
                        *y++ = dl * (float)((g >> (8 * j)) & 0xFF) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                }
            }
        }
        return 0;
    case ORC_IQ3_XXS:   /* sabah_rt.cu:2320-2344; quants.py:1039-1075 */
        for (int b = 0; b < k / 256; ++b, x += 98) {
            const float d = ld_f16(x);
            const uint8_t *qs = x + 2, *ss = x + 66;
            for (int ib = 0; ib < 8; ++ib) {
                uint32_t aux;
                memcpy(&aux, ss + 4 * ib, 4);
                const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
                for (int l = 0; l < 4; ++l) {
                    const uint8_t sg = orc_ksigns_iq2xs[(aux >> (7 * l)) & 127];
                    const uint32_t g1 = orc_iq3xxs_grid[qs[8 * ib + 2 * l]], g2 = orc_iq3xxs_grid[qs[8 * ib + 2 * l + 1]];
                    for (int j = 0; j < 4; ++j) {
                        y[j] = db * (float)((g1 >> (8 * j)) & 0xFF) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                        y[j + 4] = db * (float)((g2 >> (8 * j)) & 0xFF) * ((sg >> (j + 4)) & 1 ? -1.0f : 1.0f);
                    }
                    y += 8;
                }
            }
        }
        return 0;
    case ORC_IQ4_NL:    /* sabah_rt.cu:2380-2389; quants.py:1364-1382 */
        for (int b = 0; b < k / 32; ++b, x += 18) {
            const float d = ld_f16(x);
            for (int j = 0; j < 16; ++j) {
                y[j] = d * (float)orc_kvalues_iq4nl[x[2 + j] & 0xF];
                y[j + 16] = d * (float)orc_kvalues_iq4nl[x[2 + j] >> 4];
            }
            y += 32;
        }
        return 0;
    case ORC_Q2_0:      /* sabah_rt.cu:2411-2419; quants.py:224-235: (q - 1) * d */
        for (int b = 0; b < k / 64; ++b, x += 18) {
            const float d = ld_f16(x);
            for (int j = 0; j < 64; ++j) y[j] = (float)(((x[2 + j / 4] >> (2 * (j % 4))) & 3) - 1) * d;
            y += 64;
        }
        return 0;
    case ORC_IQ4_XS:    /* sabah_rt.cu:2391-2409; quants.py:1385-1411 */
        for (int b = 0; b < k / 256; ++b, x += 136) {
            const float d = ld_f16(x);
            const int sh = x[2] | (x[3] << 8);
            const uint8_t *sl = x + 4, *qs = x + 8;
            for (int ib = 0; ib < 8; ++ib) {
                const int ls = ((sl[ib / 2] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                for (int j = 0; j < 16; ++j) {
                    y[j] = dl * (float)orc_kvalues_iq4nl[qs[j] & 0xF];
                    y[j + 16] = dl * (float)orc_kvalues_iq4nl[qs[j] >> 4];
                }
                y += 32;
                qs += 16;
            }
        }
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------ */
/* block dots                                                                */
/* ------------------------------------------------------------------------ */

/* ggml_vec_dot_q8_0_q8_0: exact int32 per 32-block, sumf += sumi*(dw*dx). */
static float dot_q8_0(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 32; ++b, w += 34, a += 34) {
        int sumi = 0;
        for (int j = 0; j < 32; ++j) sumi += (int)(int8_t)w[2 + j] * (int)(int8_t)a[2 + j];
        sumf += (float)sumi * (ld_f16(w) * ld_f16(a));
    }
    return sumf;
}

static inline float q8K_d(const uint8_t *a) { float d; memcpy(&d, a, 4); return d; }
static inline const int8_t *q8K_qs(const uint8_t *a) { return (const int8_t *)(a + 4); }
static inline int q8K_bsum(const uint8_t *a, int j) { int16_t v; memcpy(&v, a + 260 + 2 * j, 2); return v; }

/* ggml_vec_dot_q4_K_q8_K (generic): eight int32 lanes of scale*sum(q4*q8),
 * one fp32 lane sum per lane; the min term sum(bsums*mins) is subtracted per
 * super-block with dmin*d8; lanes are added last. */
static float dot_q4_K(const uint8_t *w, const uint8_t *a, int k) {
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 144, a += 292) {
        int8_t v[256];
        const uint8_t *q = w + 16;
        for (int c = 0; c < 4; ++c, q += 32)
            for (int l = 0; l < 32; ++l) { v[64 * c + l] = (int8_t)(q[l] & 0xF); v[64 * c + 32 + l] = (int8_t)(q[l] >> 4); }
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) scale_min_k4(j, w + 4, &sc[j], &mn[j]);
        int msum = 0;
        for (int j = 0; j < 16; ++j) msum += q8K_bsum(a, j) * mn[j / 2];
        const int8_t *q8 = q8K_qs(a);
        int aux[8] = {0};
        for (int j = 0; j < 8; ++j)
            for (int m = 0; m < 4; ++m)
                for (int l = 0; l < 8; ++l) {
                    const int e = 32 * j + 8 * m + l;
                    aux[l] += sc[j] * ((int)q8[e] * (int)v[e]);
                }
        const float d = ld_f16(w) * q8K_d(a);
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux[l];
        const float dmin = ld_f16(w + 2) * q8K_d(a);
        sumf -= dmin * (float)msum;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_q5_1_q8_1 (generic): per 32-block the exact int32 sum of
 * q5 * q8, then sumf += (d_w * d_x) * sumi + m_w * s_x, blocks in order. */
static float dot_q5_1(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 32; ++b, w += 24, a += 36) {
        const uint32_t qh = (uint32_t)w[4] | ((uint32_t)w[5] << 8) | ((uint32_t)w[6] << 16) | ((uint32_t)w[7] << 24);
        const int8_t *q8 = (const int8_t *)(a + 4);
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < 16; ++j) {
            const int x0 = (w[8 + j] & 0xF) | (int)(((qh >> j) & 1u) << 4);
            const int x1 = (w[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
            sumi0 += x0 * q8[j];
            sumi1 += x1 * q8[j + 16];
        }
        const int sumi = sumi0 + sumi1;
        sumf += (ld_f16(w) * ld_f16(a)) * (float)sumi + ld_f16(w + 2) * ld_f16(a + 2);
    }
    return sumf;
}

/* ggml_vec_dot_q5_K_q8_K (generic): the q4_K lanes with each value's fifth
 * bit (qh) added; the same eight int32 lanes, fp32 lane sums and min term. */
static float dot_q5_K(const uint8_t *w, const uint8_t *a, int k) {
    float sums[8] = {0};
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 176, a += 292) {
        int8_t v[256];
        const uint8_t *q = w + 48, *hm = w + 16;
        for (int c = 0; c < 4; ++c, q += 32)
            for (int l = 0; l < 32; ++l) {
                v[64 * c + l] = (int8_t)((q[l] & 0xF) + ((hm[l] >> (2 * c)) & 1) * 16);
                v[64 * c + 32 + l] = (int8_t)((q[l] >> 4) + ((hm[l] >> (2 * c + 1)) & 1) * 16);
            }
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) scale_min_k4(j, w + 4, &sc[j], &mn[j]);
        int msum = 0;
        for (int j = 0; j < 16; ++j) msum += q8K_bsum(a, j) * mn[j / 2];
        const int8_t *q8 = q8K_qs(a);
        int aux[8] = {0};
        for (int j = 0; j < 8; ++j)
            for (int m = 0; m < 4; ++m)
                for (int l = 0; l < 8; ++l) {
                    const int e = 32 * j + 8 * m + l;
                    aux[l] += sc[j] * ((int)q8[e] * (int)v[e]);
                }
        const float d = ld_f16(w) * q8K_d(a);
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux[l];
        const float dmin = ld_f16(w + 2) * q8K_d(a);
        sumf -= dmin * (float)msum;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_q6_K_q8_K (generic): signed 6-bit values (q-32), eight int32
 * lanes of scale16*sum(q6*q8), fp32 lane sums, lanes added last. */
static float dot_q6_K(const uint8_t *w, const uint8_t *a, int k) {
    float sums[8] = {0};
    for (int b = 0; b < k / 256; ++b, w += 210, a += 292) {
        int8_t v[256];
        const uint8_t *ql = w, *qh = w + 128;
        for (int half = 0; half < 2; ++half, ql += 64, qh += 32)
            for (int l = 0; l < 32; ++l) {
                v[128 * half + l] = (int8_t)(((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                v[128 * half + 32 + l] = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                v[128 * half + 64 + l] = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                v[128 * half + 96 + l] = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
        const int8_t *sc = (const int8_t *)(w + 192);
        const int8_t *q8 = q8K_qs(a);
        int aux[8] = {0};
        for (int j = 0; j < 16; ++j)
            for (int m = 0; m < 2; ++m)
                for (int l = 0; l < 8; ++l) {
                    const int e = 16 * j + 8 * m + l;
                    aux[l] += (int)sc[j] * ((int)q8[e] * (int)v[e]);
                }
        const float d = ld_f16(w + 208) * q8K_d(a);
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux[l];
    }
    float sumf = 0.0f;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_iq3_s_q8_K (generic): per super-block the exact int32
 * bsum = sum_ib32 (2*scale+1) * sum(grid*sign*q8); sumf += (dw*d8) * bsum. */
static float dot_iq3_s(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 110, a += 292) {
        const uint8_t *qs = w + 2, *qh = w + 66, *signs = w + 74, *scales = w + 106;
        const int8_t *q8 = q8K_qs(a);
        int bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = 2 * ((scales[ib / 2] >> (4 * (ib & 1))) & 0xF) + 1;
            int sumi = 0;
            for (int g = 0; g < 8; ++g) {
                const uint32_t gi = (uint32_t)qs[8 * ib + g] | (((uint32_t)(qh[ib] >> g) & 1u) << 8);
                const uint32_t grid = orc_iq3s_grid[gi];
                const uint8_t sg = signs[4 * ib + g / 2];
                for (int j = 0; j < 4; ++j) {
                    const int mag = (int)((grid >> (8 * j)) & 0xFF);
                    const int s = (sg >> ((g & 1) * 4 + j)) & 1 ? -1 : 1;
                    sumi += mag * (int)q8[32 * ib + 4 * g + j] * s;
                }
            }
            bsum += sumi * ls;
        }
        const float d = ld_f16(w) * q8K_d(a);
        sumf += d * (float)bsum;
    }
    return sumf;
}

/* ggml_vec_dot_iq3_xxs_q8_K (generic): bsum = sum_ib32 (2*(aux>>28)+1) *
 * sum(grid*sign*q8) per super-block (sign byte = ksigns[7-bit index]);
 * sumf += (dw*d8) * bsum; the result is 0.25f * sumf. */
static float dot_iq3_xxs(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 98, a += 292) {
        const uint8_t *q3 = w + 2, *gas = w + 66;
        const int8_t *q8 = q8K_qs(a);
        int bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t aux;
            memcpy(&aux, gas + 4 * ib, 4);
            const int ls = 2 * (int)(aux >> 28) + 1;
            int sumi = 0;
            for (int l = 0; l < 4; ++l) {
                const uint32_t g1 = orc_iq3xxs_grid[q3[8 * ib + 2 * l]], g2 = orc_iq3xxs_grid[q3[8 * ib + 2 * l + 1]];
                const uint8_t sg = orc_ksigns_iq2xs[(aux >> (7 * l)) & 127];
                for (int j = 0; j < 4; ++j) {
                    sumi += (int)((g1 >> (8 * j)) & 0xFF) * (int)q8[32 * ib + 8 * l + j] * ((sg >> j) & 1 ? -1 : 1);
                    sumi += (int)((g2 >> (8 * j)) & 0xFF) * (int)q8[32 * ib + 8 * l + 4 + j] * ((sg >> (j + 4)) & 1 ? -1 : 1);
                }
            }
            bsum += sumi * ls;
        }
        const float d = ld_f16(w) * q8K_d(a);
        sumf += d * (float)bsum;
    }
    return 0.25f * sumf;
}

/* ggml_vec_dot_iq2_s_q8_K (generic): bsum = sum_ib32 (ls1 * sumi1 + ls2 * sumi2),
 * ls = 2 * nibble + 1 for the sub-block's first / second 16 elements, sumi =
 * sum(grid * sign * q8); sumf += (dw * d8) * bsum per super-block; the result
 * is 0.125f * sumf (db = d * (0.5 + nibble) * 0.25 = d * ls / 8). */
static float dot_iq2_s(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 82, a += 292) {
        const uint8_t *qs = w + 2, *signs = w + 34, *qh = w + 66, *sc = w + 74;
        const int8_t *q8 = q8K_qs(a);
        int bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const int ls1 = 1 + 2 * (sc[ib] & 0xF), ls2 = 1 + 2 * (sc[ib] >> 4);
            int sumi[2] = {0, 0};
            for (int l = 0; l < 4; ++l) {
                const uint64_t g = orc_iq2s_grid[qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300)];
                for (int j = 0; j < 8; ++j)
                    sumi[l >> 1] += (int)q8[32 * ib + 8 * l + j] * (int)((g >> (8 * j)) & 0xFF) *
                                    ((signs[4 * ib + l] >> j) & 1 ? -1 : 1);
            }
            bsum += ls1 * sumi[0] + ls2 * sumi[1];
        }
        const float d = ld_f16(w) * q8K_d(a);
        sumf += d * (float)bsum;
    }
    return 0.125f * sumf;
}

/* ggml_vec_dot_iq4_nl_q8_0 (generic): per 32-block sumf += (d8*dw) * sum(kv[q]*q8). */
static float dot_iq4_nl(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 32; ++b, w += 18, a += 34) {
        const float d = ld_f16(a) * ld_f16(w);
        const int8_t *q8 = (const int8_t *)(a + 2);
        int s1 = 0, s2 = 0;
        for (int j = 0; j < 16; ++j) {
            s1 += (int)q8[j] * (int)orc_kvalues_iq4nl[w[2 + j] & 0xF];
            s2 += (int)q8[j + 16] * (int)orc_kvalues_iq4nl[w[2 + j] >> 4];
        }
        sumf += d * (float)(s1 + s2);
    }
    return sumf;
}

/* Q2_0 x q8_0.  ggml's CPU source for this type is not in the reference, so
 * the activation type and the float order are a choice (parity unpinned for
 * them): q8_0 activations, as ggml pairs its other 32-element-grouped legacy
 * formats, and per 32-element half of a 64-element block, in element order,
 * sumf += (float)sumi * (d_w * d_8), the form of ggml_vec_dot_q8_0_q8_0.
 * The codes and their offset follow the reference's decoders
 * (sabah_rt.cu:2411-2419 host, 2547-2557 device). */
static float dot_q2_0(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 64; ++b, w += 18) {
        const float dw = ld_f16(w);
        for (int h = 0; h < 2; ++h, a += 34) {
            const int8_t *q8 = (const int8_t *)(a + 2);
            int sumi = 0;
            for (int j = 0; j < 32; ++j) {
                const int e = 32 * h + j;
                sumi += (int)q8[j] * (((w[2 + e / 4] >> (2 * (e % 4))) & 3) - 1);
            }
            sumf += (float)sumi * (dw * ld_f16(a));
        }
    }
    return sumf;
}

/* ggml_vec_dot_iq4_xs_q8_K (generic): per 32-element sub-block
 * sumf += ((dw*d8) * (ls - 32)) * sum(kv[q]*q8), sub-blocks in order. */
static float dot_iq4_xs(const uint8_t *w, const uint8_t *a, int k) {
    float sumf = 0.0f;
    for (int b = 0; b < k / 256; ++b, w += 136, a += 292) {
        const float d4d8 = ld_f16(w) * q8K_d(a);
        const int sh = w[2] | (w[3] << 8);
        const uint8_t *sl = w + 4, *qs = w + 8;
        const int8_t *q8 = q8K_qs(a);
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = ((sl[ib / 2] >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
            const float dl = d4d8 * (float)(ls - 32);
            int s1 = 0, s2 = 0;
            for (int j = 0; j < 16; ++j) {
                s1 += (int)q8[32 * ib + j] * (int)orc_kvalues_iq4nl[qs[16 * ib + j] & 0xF];
                s2 += (int)q8[32 * ib + 16 + j] * (int)orc_kvalues_iq4nl[qs[16 * ib + j] >> 4];
            }
            sumf += dl * (float)(s1 + s2);
        }
    }
    return sumf;
}

float orc_vec_dot(int qt, const uint8_t *w, const uint8_t *a, int k) {
    switch (qt) {
    case ORC_Q8_0: return dot_q8_0(w, a, k);
    case ORC_Q5_1: return dot_q5_1(w, a, k);
    case ORC_Q4_K: return dot_q4_K(w, a, k);
    case ORC_Q5_K: return dot_q5_K(w, a, k);
    case ORC_Q6_K: return dot_q6_K(w, a, k);
    case ORC_IQ3_S: return dot_iq3_s(w, a, k);
    case ORC_IQ3_XXS: return dot_iq3_xxs(w, a, k);
    case ORC_IQ2_S: return dot_iq2_s(w, a, k);
    case ORC_IQ4_NL: return dot_iq4_nl(w, a, k);
    case ORC_IQ4_XS: return dot_iq4_xs(w, a, k);
    case ORC_Q2_0: return dot_q2_0(w, a, k);
    }
    return NAN;
}

/* ------------------------------------------------------------------------ */
/* weight encoders (synthetic data)                                           */
/* ------------------------------------------------------------------------ */
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

/* nearest codebook entry for every 4-tuple of 3-bit levels (squared level distance,
 * lowest index on ties) */
static uint16_t g_iq3s_nearest[4096];
static int g_iq3s_nearest_ready = 0;

static void iq3s_nearest_init(void) {
    if (g_iq3s_nearest_ready) return;
    for (int key = 0; key < 4096; ++key) {
        int best = 0, bestd = 1 << 30;
        for (int e = 0; e < 512; ++e) {
            int dist = 0;
            for (int j = 0; j < 4; ++j) {
                const int lv = (key >> (3 * j)) & 7;
                const int ge = (int)((orc_iq3s_grid[e] >> (8 * j)) & 0xFF) / 2;
                dist += (lv - ge) * (lv - ge);
            }
            if (dist < bestd) { bestd = dist; best = e; }
        }
        g_iq3s_nearest[key] = (uint16_t)best;
    }
    g_iq3s_nearest_ready = 1;
}

static void enc_iq3_s(const float *x, uint8_t *y, int k) {
    iq3s_nearest_init();
    for (int b = 0; b < k / 256; ++b, x += 256, y += 110) {
        memset(y, 0, 110);
        float am[8], A = 0.0f;
        for (int ib = 0; ib < 8; ++ib) {
            am[ib] = 0.0f;
            for (int j = 0; j < 32; ++j) am[ib] = fmaxf(am[ib], fabsf(x[32 * ib + j]));
            A = fmaxf(A, am[ib]);
        }
        if (A == 0.0f) continue;
        st_f16(y, A / 465.0f);
        const float df = ld_f16(y);
        if (df == 0.0f) { memset(y, 0, 110); continue; }
        uint8_t *qs = y + 2, *qh = y + 66, *signs = y + 74, *scales = y + 106;
        for (int ib = 0; ib < 8; ++ib) {
            const int s = clampi((int)lrintf((am[ib] / (15.0f * df) - 1.0f) * 0.5f), 0, 15);
            const float dl = df * (float)(2 * s + 1);
            scales[ib / 2] |= (uint8_t)(s << (4 * (ib & 1)));
            for (int g = 0; g < 8; ++g) {
                int key = 0;
                for (int j = 0; j < 4; ++j) {
                    const float v = x[32 * ib + 4 * g + j];
                    const int lv = clampi((int)lrintf((fabsf(v) / dl - 1.0f) * 0.5f), 0, 7);
                    key |= lv << (3 * j);
                    if (v < 0.0f) signs[4 * ib + g / 2] |= (uint8_t)(1u << ((g & 1) * 4 + j));
                }
                const int gi = g_iq3s_nearest[key];
                qs[8 * ib + g] = (uint8_t)(gi & 0xFF);
                qh[ib] |= (uint8_t)((gi >> 8) << g);
            }
        }
    }
}

static void enc_q4_K(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 256; ++b, x += 256, y += 144) {
        memset(y, 0, 144);
        float scl[8], mns[8], msc = 0.0f, mmn = 0.0f;
        for (int j = 0; j < 8; ++j) {
            float lo = 0.0f, hi = 0.0f;
            for (int l = 0; l < 32; ++l) { lo = fminf(lo, x[32 * j + l]); hi = fmaxf(hi, x[32 * j + l]); }
            scl[j] = (hi - lo) / 15.0f;
            mns[j] = -lo;
            msc = fmaxf(msc, scl[j]);
            mmn = fmaxf(mmn, mns[j]);
        }
        st_f16(y, msc / 63.0f);
        st_f16(y + 2, mmn / 63.0f);
        const float df = ld_f16(y), dmf = ld_f16(y + 2);
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = df > 0.0f ? clampi((int)lrintf(scl[j] / df), 0, 63) : 0;
            mn[j] = dmf > 0.0f ? clampi((int)lrintf(mns[j] / dmf), 0, 63) : 0;
        }
        uint8_t *p = y + 4;
        for (int j = 0; j < 4; ++j) {
            p[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            p[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
            p[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; ++j) {
            const float step = df * (float)sc[j], off = dmf * (float)mn[j];
            for (int l = 0; l < 32; ++l)
                q[32 * j + l] = (uint8_t)(step > 0.0f ? clampi((int)lrintf((x[32 * j + l] + off) / step), 0, 15) : 0);
        }
        uint8_t *qs = y + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l) qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
    }
}

/* Q5_1: per 32-block the range [min, max] in 31 steps (ggml's
 * quantize_row_q5_1_ref steps: d = (max - min) / 31, m = min, q = x / d -
 * m / d rounded half up, clamped to 31) */
static void enc_q5_1(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 32; ++b, x += 32, y += 24) {
        float lo = x[0], hi = x[0];
        for (int j = 1; j < 32; ++j) { lo = fminf(lo, x[j]); hi = fmaxf(hi, x[j]); }
        const float d = (hi - lo) / 31.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        st_f16(y, d);
        st_f16(y + 2, lo);
        uint32_t qh = 0;
        for (int j = 0; j < 16; ++j) {
            const int q0 = clampi((int)((x[j] - lo) * id + 0.5f), 0, 31);
            const int q1 = clampi((int)((x[j + 16] - lo) * id + 0.5f), 0, 31);
            y[8 + j] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
            qh |= ((uint32_t)(q0 >> 4) << j) | ((uint32_t)(q1 >> 4) << (j + 16));
        }
        memcpy(y + 4, &qh, 4);
    }
}

/* Q5_K: enc_q4_K's scales and mins with 31 levels per sub-block and the fifth
 * bit in qh (this project's encoder; any valid bytes serve the parity tests) */
static void enc_q5_K(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 256; ++b, x += 256, y += 176) {
        memset(y, 0, 176);
        float scl[8], mns[8], msc = 0.0f, mmn = 0.0f;
        for (int j = 0; j < 8; ++j) {
            float lo = 0.0f, hi = 0.0f;
            for (int l = 0; l < 32; ++l) { lo = fminf(lo, x[32 * j + l]); hi = fmaxf(hi, x[32 * j + l]); }
            scl[j] = (hi - lo) / 31.0f;
            mns[j] = -lo;
            msc = fmaxf(msc, scl[j]);
            mmn = fmaxf(mmn, mns[j]);
        }
        st_f16(y, msc / 63.0f);
        st_f16(y + 2, mmn / 63.0f);
        const float df = ld_f16(y), dmf = ld_f16(y + 2);
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = df > 0.0f ? clampi((int)lrintf(scl[j] / df), 0, 63) : 0;
            mn[j] = dmf > 0.0f ? clampi((int)lrintf(mns[j] / dmf), 0, 63) : 0;
        }
        uint8_t *p = y + 4;
        for (int j = 0; j < 4; ++j) {
            p[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            p[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
            p[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
        }
        uint8_t *qh = y + 16, *qs = y + 48;
        for (int j = 0; j < 8; ++j) {
            const float step = df * (float)sc[j], off = dmf * (float)mn[j];
            for (int l = 0; l < 32; ++l) {
                const int q = step > 0.0f ? clampi((int)lrintf((x[32 * j + l] + off) / step), 0, 31) : 0;
                qs[32 * (j / 2) + l] |= (uint8_t)((q & 0xF) << (4 * (j & 1)));
                qh[l] |= (uint8_t)((q >> 4) << j);
            }
        }
    }
}

static void enc_q6_K(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 256; ++b, x += 256, y += 210) {
        memset(y, 0, 210);
        float scl[16], ms = 0.0f;
        for (int j = 0; j < 16; ++j) {
            float am = 0.0f;
            for (int l = 0; l < 16; ++l) am = fmaxf(am, fabsf(x[16 * j + l]));
            scl[j] = am / 31.0f;
            ms = fmaxf(ms, scl[j]);
        }
        st_f16(y + 208, ms / 127.0f);
        const float df = ld_f16(y + 208);
        int8_t *sc = (int8_t *)(y + 192);
        uint8_t u[256];
        for (int j = 0; j < 16; ++j) {
            sc[j] = (int8_t)(df > 0.0f ? clampi((int)lrintf(scl[j] / df), -128, 127) : 0);
            const float step = df * (float)sc[j];
            for (int l = 0; l < 16; ++l) {
                const int q = step != 0.0f ? clampi((int)lrintf(x[16 * j + l] / step), -32, 31) : 0;
                u[16 * j + l] = (uint8_t)(q + 32);
            }
        }
        uint8_t *ql = y, *qh = y + 128;
        for (int half = 0; half < 2; ++half)
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = u[128 * half + l], q2 = u[128 * half + 32 + l];
                const uint8_t q3 = u[128 * half + 64 + l], q4 = u[128 * half + 96 + l];
                ql[64 * half + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[64 * half + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[32 * half + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
    }
}

/* IQ4 levels: the index of the level nearest v (lowest on ties) */
static int iq4_nearest(float v) {
    int best = 0;
    float be = fabsf(v - (float)orc_kvalues_iq4nl[0]);
    for (int i = 1; i < 16; ++i) {
        const float e = fabsf(v - (float)orc_kvalues_iq4nl[i]);
        if (e < be) { be = e; best = i; }
    }
    return best;
}

/* simple IQ4_NL encoder (synthetic data): d = amax / 127 per 32-block, nearest level */
static void enc_iq4_nl(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 32; ++b, x += 32, y += 18) {
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const uint16_t dh = orc_fp32_to_fp16(amax / 127.0f);
        const float d = orc_fp16_to_fp32(dh), id = d > 0.0f ? 1.0f / d : 0.0f;
        y[0] = (uint8_t)dh; y[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 16; ++j)
            y[2 + j] = (uint8_t)(iq4_nearest(x[j] * id) | (iq4_nearest(x[j + 16] * id) << 4));
    }
}

/* simple IQ4_XS encoder (synthetic data): one fp16 d per super-block, 6-bit
 * sub-block scales ls in [33, 63] (ls - 32 in [1, 31]), nearest level */
static void enc_iq4_xs(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 256; ++b, x += 256, y += 136) {
        float am[8], amax = 0.0f;
        for (int ib = 0; ib < 8; ++ib) {
            am[ib] = 0.0f;
            for (int j = 0; j < 32; ++j) am[ib] = fmaxf(am[ib], fabsf(x[32 * ib + j]));
            amax = fmaxf(amax, am[ib]);
        }
        const uint16_t dh = orc_fp32_to_fp16(amax / (127.0f * 31.0f));
        const float d = orc_fp16_to_fp32(dh);
        y[0] = (uint8_t)dh; y[1] = (uint8_t)(dh >> 8);
        memset(y + 2, 0, 6);
        int sh = 0;
        for (int ib = 0; ib < 8; ++ib) {
            const int s = d > 0.0f ? clampi((int)lrintf(am[ib] / (127.0f * d)), 1, 31) : 1;
            const int ls = s + 32;
            y[4 + ib / 2] |= (uint8_t)((ls & 0xF) << (4 * (ib & 1)));
            sh |= ((ls >> 4) & 3) << (2 * ib);
            const float id = d > 0.0f ? 1.0f / (d * (float)s) : 0.0f;
            for (int j = 0; j < 16; ++j)
                y[8 + 16 * ib + j] = (uint8_t)(iq4_nearest(x[32 * ib + j] * id) |
                                               (iq4_nearest(x[32 * ib + 16 + j] * id) << 4));
        }
        y[2] = (uint8_t)sh; y[3] = (uint8_t)(sh >> 8);
    }
}

/* simple Q2_0 encoder (synthetic data): d = amax / 2 per 64-block, nearest of
 * (q - 1) * d for q in 0..3 */
static void enc_q2_0(const float *x, uint8_t *y, int k) {
    for (int b = 0; b < k / 64; ++b, x += 64, y += 18) {
        float amax = 0.0f;
        for (int j = 0; j < 64; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const uint16_t dh = orc_fp32_to_fp16(amax / 2.0f);
        const float d = orc_fp16_to_fp32(dh), id = d > 0.0f ? 1.0f / d : 0.0f;
        y[0] = (uint8_t)dh; y[1] = (uint8_t)(dh >> 8);
        memset(y + 2, 0, 16);
        for (int j = 0; j < 64; ++j)
            y[2 + j / 4] |= (uint8_t)(clampi((int)lrintf(x[j] * id) + 1, 0, 3) << (2 * (j % 4)));
    }
}

int orc_quantize_weights(int qt, const float *x, uint8_t *y, int k) {
    if (orc_row_bytes(qt, k) == 0) return -1;
    switch (qt) {
    case ORC_Q8_0: orc_quantize_q8_0(x, y, k); return 0;
    case ORC_Q4_K: enc_q4_K(x, y, k); return 0;
    case ORC_Q5_1: enc_q5_1(x, y, k); return 0;
    case ORC_Q5_K: enc_q5_K(x, y, k); return 0;
    case ORC_Q6_K: enc_q6_K(x, y, k); return 0;
    case ORC_IQ3_S: enc_iq3_s(x, y, k); return 0;
    case ORC_IQ4_NL: enc_iq4_nl(x, y, k); return 0;
    case ORC_IQ4_XS: enc_iq4_xs(x, y, k); return 0;
    case ORC_Q2_0: enc_q2_0(x, y, k); return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------------ */
/* MUL_MAT_ID                                                                */
/* ------------------------------------------------------------------------ */
static int threads_or_default(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

int orc_mul_mat_id(const void *source, size_t expert_stride, size_t row_stride,
                   const float *x, size_t x_id_stride, int x_rows, size_t x_token_stride,
                   const int32_t *ids, size_t ids_id_stride, size_t ids_token_stride,
                   int n_ids, int n_tokens,
                   float *dst, size_t dst_id_stride, size_t dst_token_stride,
                   int rows, int k, int n_experts, int qt, int n_threads) {
    if (n_tokens == 0) return 0;
    const size_t rb = orc_row_bytes(qt, k);
    const size_t ab = orc_act_row_bytes(qt, k);
    if (!source || !x || !ids || !dst || rb == 0 || ab == 0 || row_stride < rb || rows <= 0 ||
        n_ids <= 0 || n_tokens < 0 || n_experts <= 0 || (x_rows != 1 && x_rows != n_ids))
        return -1;
    for (int t = 0; t < n_tokens; ++t)
        for (int i = 0; i < n_ids; ++i) {
            const int32_t e = *(const int32_t *)((const uint8_t *)ids + (size_t)t * ids_token_stride + (size_t)i * ids_id_stride);
            if (e < 0 || e >= n_experts) return -1;
        }
    /* src1 -> vec_dot_type, once per input row (as ggml converts all of src1 first) */
    uint8_t *act = (uint8_t *)malloc(ab * (size_t)n_tokens * (size_t)x_rows);
    if (!act) return -1;
    const int nt = threads_or_default(n_threads);
    #pragma omp parallel for num_threads(nt) schedule(static)
    for (int p = 0; p < n_tokens * x_rows; ++p) {
        const int t = p / x_rows, r = p % x_rows;
        const float *xr = (const float *)((const uint8_t *)x + (size_t)t * x_token_stride + (size_t)r * x_id_stride);
        orc_quantize_act(qt, xr, act + (size_t)p * ab, k);
    }
    const long total = (long)n_tokens * n_ids * rows;
    #pragma omp parallel for num_threads(nt) schedule(static)
    for (long q = 0; q < total; ++q) {
        const int r = (int)(q % rows);
        const int i = (int)((q / rows) % n_ids);
        const int t = (int)(q / ((long)rows * n_ids));
        const int32_t e = *(const int32_t *)((const uint8_t *)ids + (size_t)t * ids_token_stride + (size_t)i * ids_id_stride);
        const uint8_t *w = (const uint8_t *)source + (size_t)e * expert_stride + (size_t)r * row_stride;
        const uint8_t *a = act + ((size_t)t * x_rows + (size_t)(i % x_rows)) * ab;
        float *o = (float *)((uint8_t *)dst + (size_t)t * dst_token_stride + (size_t)i * dst_id_stride) + r;
        *o = orc_vec_dot(qt, w, a, k);
    }
    free(act);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* one MoE layer (gated FFN of the routed experts + optional shared expert)  */
/* ------------------------------------------------------------------------ */
static inline float silu_f32(float v) { return v / (1.0f + expf(-v)); }

/* One MoE layer as ggml's graph computes it (qwen4exp.cpp:848-892): x
 * quantised to the gate/up vec_dot type once per token; the gate and up
 * MUL_MAT_IDs over every (token, slot, row); h = silu(g) * u; h quantised to
 * the down vec_dot type once per (token, slot); the down MUL_MAT_ID; then per
 * token the router-weighted sum over the slots in slot order and the
 * (optionally sigmoid-gated) shared expert.  The phases run inside one
 * OpenMP parallel region (one fork per call); every value is computed by one
 * thread in the order stated, so the result does not depend on the thread
 * count. */
int orc_moe_layer(const orc_moe_layer_desc *L, const float *x, const int32_t *ids,
                  const float *w, int n_used, int n_tokens, float *out, float *h_out, int n_threads) {
    const int D = L->d_model, F = L->d_ff, T = n_tokens, K = n_used;
    const size_t rbg = orc_row_bytes(L->qt_gate, D), rbu = orc_row_bytes(L->qt_up, D);
    const size_t rbd = orc_row_bytes(L->qt_down, F);
    if (!rbg || !rbu || !rbd || K <= 0 || T < 0) return -1;
    for (int p = 0; p < T * K; ++p)
        if (ids[p] < 0 || ids[p] >= L->n_experts) return -1;
    if (T == 0) return 0;
    const int nt = threads_or_default(n_threads);
    const size_t esg = rbg * (size_t)F, esu = rbu * (size_t)F, esd = rbd * (size_t)D;
    const size_t abg = orc_act_row_bytes(L->qt_gate, D), abu = orc_act_row_bytes(L->qt_up, D);
    const size_t abd = orc_act_row_bytes(L->qt_down, F);
    const int P = T * K;
    const int Fs = L->shared_gate ? L->d_ff_shared : 0;
    const size_t abs_g = Fs ? orc_act_row_bytes(L->qt_shared_gate, D) : 0;
    const size_t abs_u = Fs ? orc_act_row_bytes(L->qt_shared_up, D) : 0;
    const size_t abs_d = Fs ? orc_act_row_bytes(L->qt_shared_down, Fs) : 0;
    const size_t rbs_g = Fs ? orc_row_bytes(L->qt_shared_gate, D) : 0, rbs_u = Fs ? orc_row_bytes(L->qt_shared_up, D) : 0;
    const size_t rbs_d = Fs ? orc_row_bytes(L->qt_shared_down, Fs) : 0;
    uint8_t *xg = (uint8_t *)malloc(abg * (size_t)T), *xu = (uint8_t *)malloc(abu * (size_t)T);
    float *g = (float *)malloc(sizeof(float) * (size_t)P * F), *u = (float *)malloc(sizeof(float) * (size_t)P * F);
    uint8_t *hq = (uint8_t *)malloc(abd * (size_t)P);
    float *y = (float *)malloc(sizeof(float) * (size_t)P * D);
    uint8_t *xsg = Fs ? (uint8_t *)malloc(abs_g * (size_t)T) : NULL, *xsu = Fs ? (uint8_t *)malloc(abs_u * (size_t)T) : NULL;
    float *gs = Fs ? (float *)malloc(sizeof(float) * (size_t)T * Fs) : NULL;
    float *us = Fs ? (float *)malloc(sizeof(float) * (size_t)T * Fs) : NULL;
    uint8_t *hsq = Fs ? (uint8_t *)malloc(abs_d * (size_t)T) : NULL;
    float *ys = Fs ? (float *)malloc(sizeof(float) * (size_t)T * D) : NULL;
    #pragma omp parallel num_threads(nt)
    {
        #pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            const float *xt = x + (size_t)t * D;
            orc_quantize_act(L->qt_gate, xt, xg + (size_t)t * abg, D);
            orc_quantize_act(L->qt_up, xt, xu + (size_t)t * abu, D);
            if (Fs) {
                orc_quantize_act(L->qt_shared_gate, xt, xsg + (size_t)t * abs_g, D);
                orc_quantize_act(L->qt_shared_up, xt, xsu + (size_t)t * abs_u, D);
            }
        }
        /* gate and up MUL_MAT_ID: (token, slot, row) */
        #pragma omp for schedule(static)
        for (long q = 0; q < (long)P * F; ++q) {
            const int p = (int)(q / F), j = (int)(q % F), t = p / K;
            const int e = ids[p];
            g[q] = orc_vec_dot(L->qt_gate, (const uint8_t *)L->gate + (size_t)e * esg + (size_t)j * rbg, xg + (size_t)t * abg, D);
            u[q] = orc_vec_dot(L->qt_up, (const uint8_t *)L->up + (size_t)e * esu + (size_t)j * rbu, xu + (size_t)t * abu, D);
        }
        if (Fs) {
            #pragma omp for schedule(static)
            for (long q = 0; q < (long)T * Fs; ++q) {
                const int t = (int)(q / Fs), j = (int)(q % Fs);
                gs[q] = orc_vec_dot(L->qt_shared_gate, (const uint8_t *)L->shared_gate + (size_t)j * rbs_g, xsg + (size_t)t * abs_g, D);
                us[q] = orc_vec_dot(L->qt_shared_up, (const uint8_t *)L->shared_up + (size_t)j * rbs_u, xsu + (size_t)t * abs_u, D);
            }
        }
        /* h = silu(g) * u (ggml_swiglu), then h -> the down vec_dot type per (token, slot) */
        #pragma omp for schedule(static)
        for (int p = 0; p < P; ++p) {
            float *hp = g + (size_t)p * F;
            const float *up = u + (size_t)p * F;
            for (int j = 0; j < F; ++j) hp[j] = silu_f32(hp[j]) * up[j];
            orc_quantize_act(L->qt_down, hp, hq + (size_t)p * abd, F);
        }
        if (Fs) {
            #pragma omp for schedule(static)
            for (int t = 0; t < T; ++t) {
                float *hp = gs + (size_t)t * Fs;
                const float *up = us + (size_t)t * Fs;
                for (int j = 0; j < Fs; ++j) hp[j] = silu_f32(hp[j]) * up[j];
                orc_quantize_act(L->qt_shared_down, hp, hsq + (size_t)t * abs_d, Fs);
            }
        }
        /* down MUL_MAT_ID: (token, slot, row) */
        #pragma omp for schedule(static)
        for (long q = 0; q < (long)P * D; ++q) {
            const int p = (int)(q / D), i = (int)(q % D);
            y[q] = orc_vec_dot(L->qt_down, (const uint8_t *)L->down + (size_t)ids[p] * esd + (size_t)i * rbd,
                               hq + (size_t)p * abd, F);
        }
        if (Fs) {
            #pragma omp for schedule(static)
            for (long q = 0; q < (long)T * D; ++q) {
                const int t = (int)(q / D), i = (int)(q % D);
                ys[q] = orc_vec_dot(L->qt_shared_down, (const uint8_t *)L->shared_down + (size_t)i * rbs_d,
                                    hsq + (size_t)t * abs_d, Fs);
            }
        }
        /* combine: sum over the slots in slot order, then the shared expert */
        #pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            float *ot = out + (size_t)t * D;
            const float *yt = y + (size_t)t * K * D;
            for (int i = 0; i < D; ++i) {
                float acc = yt[i] * w[t * K + 0];
                for (int s2 = 1; s2 < K; ++s2) acc = acc + yt[(size_t)s2 * D + i] * w[t * K + s2];
                ot[i] = acc;
            }
            if (Fs) {
                const float *yst = ys + (size_t)t * D;
                float gl = 1.0f;
                if (L->shared_gate_inp) {
                    double dot = 0.0;
                    for (int i = 0; i < D; ++i) dot += (double)L->shared_gate_inp[i] * (double)x[(size_t)t * D + i];
                    gl = 1.0f / (1.0f + expf(-(float)dot));       /* ggml_vec_sigmoid_f32 */
                }
                for (int i = 0; i < D; ++i) ot[i] = ot[i] + (L->shared_gate_inp ? yst[i] * gl : yst[i]);
            }
        }
    }
    if (h_out) memcpy(h_out, g, sizeof(float) * (size_t)P * F);
    free(xg); free(xu); free(g); free(u); free(hq); free(y);
    free(xsg); free(xsu); free(gs); free(us); free(hsq); free(ys);
    return 0;
}

int orc_moe_route(const float *logits, int n_tokens, int n_experts, int n_used, int norm_w, float w_scale,
                  int32_t *ids, float *w) {
    if (n_experts <= 0 || n_used <= 0 || n_used > n_experts || n_tokens < 0) return -1;
    float *p = (float *)malloc(sizeof(float) * (size_t)n_experts);
    char *taken = (char *)malloc((size_t)n_experts);
    for (int t = 0; t < n_tokens; ++t) {
        const float *l = logits + (size_t)t * n_experts;
        float m = -INFINITY;
        for (int i = 0; i < n_experts; ++i) m = l[i] > m ? l[i] : m;           /* ggml_vec_max_f32 */
        double sum = 0.0;
        for (int i = 0; i < n_experts; ++i) {                                  /* ggml_vec_soft_max_f32 */
            p[i] = expf(l[i] - m);
            sum += (double)p[i];
        }
        const float inv = (float)(1.0 / sum);                                  /* ggml_vec_scale_f32 */
        for (int i = 0; i < n_experts; ++i) p[i] = p[i] * inv;
        memset(taken, 0, (size_t)n_experts);
        int32_t *it = ids + (size_t)t * n_used;
        float *wt = w + (size_t)t * n_used;
        for (int k = 0; k < n_used; ++k) {
            int best = -1;
            for (int i = 0; i < n_experts; ++i)
                if (!taken[i] && (best < 0 || p[i] > p[best])) best = i;
            taken[best] = 1;
            it[k] = best;
            wt[k] = p[best];
        }
        if (norm_w) {
            double d = 0.0;
            for (int k = 0; k < n_used; ++k) d += (double)wt[k];                /* ggml_vec_sum_f32 */
            const float s = (float)d;
            for (int k = 0; k < n_used; ++k) wt[k] = wt[k] / s;
        }
        if (w_scale != 1.0f)
            for (int k = 0; k < n_used; ++k) wt[k] = wt[k] * w_scale;
    }
    free(p);
    free(taken);
    return 0;
}
