// Register-resident decoding of quantised weights, one "unit" per lane.
//
// A unit is one 256-element super-block (Q4_K 144 B, Q5_K 176 B, Q6_K 210 B,
// IQ3_S 110 B, IQ3_XXS 98 B, IQ2_S 82 B, IQ4_XS 136 B), four 32-element blocks
// (Q8_0 136 B, Q5_1 96 B, IQ4_NL 72 B) or four 64-element blocks (Q2_0 72 B).  Each lane loads its unit straight
// from HBM into VGPRs with 8-byte loads that cover exactly the unit's 8-byte
// granules (so a load never touches a page the unit does not), then
// re-aligns the bytes so that every field of the format sits at a static
// dword index, and decodes with integer dot products against the unit's 256
// q8 activations held in LDS.
//
// Field origin: all fields used in the inner loops start at the same residue
// mod 4 inside the block (IQ3_S, IQ3_XXS, IQ2_S: byte 2; Q8_0 and IQ4_NL even
// blocks: byte 2; Q4_K, Q5_K, Q6_K, IQ4_XS and Q5_1: byte 0).  F[i] is the dword at
// (unit start + ORG + 4 i); Fm1 is the dword before it (the IQ formats read
// their fp16 d there).
//
// Block layouts: sabah_rt.cu:2462-2485 (Q4_K), 2487-2512 (Q5_K), 2514-2535
// (Q5_1), 2537-2545 (Q8_0), 2618-2647
// (IQ3_S), 2293-2318 (IQ2_S), 2320-2344 (IQ3_XXS), 2380-2409 (IQ4_NL,
// IQ4_XS); gguf-py
// quants.py:586-606 (Q6_K: ql[128] qh[64] int8 sc[16] d).
#pragma once
#include "quant_formats.h"

namespace sabah {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Weight loads are plain cached loads: the eight lanes that share a weight row
// read overlapping cache lines across several load instructions, and L1/L2
// must absorb those repeats.  SABAH_STREAM_LOADS=1 selects non-temporal loads.
#ifndef SABAH_STREAM_LOADS
#define SABAH_STREAM_LOADS 0
#endif
template <typename T>
__device__ inline T weight_load(const T* p) {
#if SABAH_STREAM_LOADS
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

template <int QT> struct UnitFmt;
template <> struct UnitFmt<QT_IQ3_S> { static constexpr int BYTES = 110, ELEMS = 256, ORG = 2, NF = 27, CONTRIB = 1; };
template <> struct UnitFmt<QT_Q4_K> { static constexpr int BYTES = 144, ELEMS = 256, ORG = 0, NF = 36, CONTRIB = 1; };
template <> struct UnitFmt<QT_Q6_K> { static constexpr int BYTES = 210, ELEMS = 256, ORG = 0, NF = 53, CONTRIB = 1; };
template <> struct UnitFmt<QT_Q8_0> { static constexpr int BYTES = 136, ELEMS = 128, ORG = 2, NF = 34, CONTRIB = 4; };
template <> struct UnitFmt<QT_IQ3_XXS> { static constexpr int BYTES = 98, ELEMS = 256, ORG = 2, NF = 24, CONTRIB = 1; };
template <> struct UnitFmt<QT_IQ4_XS> { static constexpr int BYTES = 136, ELEMS = 256, ORG = 0, NF = 34, CONTRIB = 8; };
template <> struct UnitFmt<QT_IQ4_NL> { static constexpr int BYTES = 72, ELEMS = 128, ORG = 2, NF = 18, CONTRIB = 4; };
template <> struct UnitFmt<QT_IQ2_S> { static constexpr int BYTES = 82, ELEMS = 256, ORG = 2, NF = 20, CONTRIB = 1; };
template <> struct UnitFmt<QT_Q2_0> { static constexpr int BYTES = 72, ELEMS = 256, ORG = 2, NF = 18, CONTRIB = 8; };
template <> struct UnitFmt<QT_Q5_K> { static constexpr int BYTES = 176, ELEMS = 256, ORG = 0, NF = 44, CONTRIB = 1; };
template <> struct UnitFmt<QT_Q5_1> { static constexpr int BYTES = 96, ELEMS = 128, ORG = 0, NF = 24, CONTRIB = 4; };

// Window: the unit's granules, loaded from base = (origin - 4) rounded down to
// 8 bytes; the origin then sits at byte p in [4, 11] of the window.
template <int QT>
struct UnitWindow {
    static constexpr int ORG = UnitFmt<QT>::ORG;
    static constexpr int NF = UnitFmt<QT>::NF;
    static constexpr int NG = (11 + UnitFmt<QT>::BYTES - ORG + 7) / 8;   // granules, worst case
    static constexpr int NW = 2 * NG + 2;                                 // dwords incl. zero tail
    uint32_t W[NW];
    int p;

    // Every load is issued unconditionally (so the compiler can count them
    // when it waits for older loads); a first or last granule that holds no
    // byte of the unit is replaced by a neighbour that does, whose bytes are
    // never read.  Only granules holding unit bytes are read, so no load
    // touches a page the unit does not.
    // len: bytes of this unit (smaller than BYTES only for the last Q8_0 unit
    // of a row that is not a whole number of 4-block units)
    __device__ inline void load(const uint8_t* unit, int len = UnitFmt<QT>::BYTES) {
        const uint8_t* o = unit + ORG;
        const int mis = (int)((reinterpret_cast<uintptr_t>(o) - 4) & 7);
        p = 4 + mis;
        const uint8_t* base = o - p;                            // 8-byte aligned
        const int first = (p - ORG < 8) ? 0 : 1;                // first granule holding unit bytes
        const int lim = len - ORG + p;                          // window offset one past the unit
        const int last = min(NG - 1, (lim - 1) >> 3);           // last granule holding unit bytes
        typedef __attribute__((address_space(1))) const u32x2 gu32x2;
        gu32x2* g = (gu32x2*)base;
        u32x2 v = weight_load(g + first);
        W[0] = v.x;
        W[1] = v.y;
#pragma unroll
        for (int i = 1; i < NG - 1; ++i) {
            v = weight_load(g + i);
            W[2 * i] = v.x;
            W[2 * i + 1] = v.y;
        }
        v = weight_load(g + last);
        W[2 * (NG - 1)] = v.x;
        W[2 * (NG - 1) + 1] = v.y;
        W[NW - 2] = W[NW - 1] = 0u;
    }

    // F[-1 .. NF-1] at static indices: select the dword shift (p >= 8), then the
    // byte shift (p & 3 in {0, 2})
    __device__ inline void fields(uint32_t (&F)[NF], uint32_t& Fm1) const {
        const bool hi = p >= 8;
        const uint32_t sh = (uint32_t)(p & 3);
        uint32_t V[NF + 2];
#pragma unroll
        for (int i = 0; i < NF + 2; ++i) V[i] = hi ? W[i + 1] : W[i];
        // origin dword index inside V is 1 (p in [4, 7]) / 2 (p in [8, 11]) -> 1 after the select
        Fm1 = __builtin_amdgcn_alignbyte(V[1], V[0], sh);
#pragma unroll
        for (int i = 0; i < NF; ++i) F[i] = __builtin_amdgcn_alignbyte(V[i + 2], V[i + 1], sh);
    }
};

// The same fields read from a unit staged in LDS: NF + 2 dwords from the
// dword-aligned address at or below (origin - 4), then one byte shift
// (origin mod 4) per field.  Bytes outside the unit are read but never used.
template <int QT>
struct LdsWindow {
    static constexpr int ORG = UnitFmt<QT>::ORG;
    static constexpr int NF = UnitFmt<QT>::NF;
    uint32_t W[NF + 2];
    uint32_t sh;
    // the address stays derived from the LDS pointer (no integer round trip),
    // so the reads are LDS instructions, not flat ones
    __device__ inline void load(const uint8_t* unit_lds) {
        // A unit whose NF dwords are exactly its bytes, at an A-aligned address
        // (A = 16 or 8, units an odd number of A-byte words apart: Q4_K 9 x 16,
        // Q8_0 / IQ4_XS 17 x 8, IQ4_NL 9 x 8 bytes), is read as A-byte words:
        // lanes on consecutive units then cover every bank, where dword reads
        // put 32 lanes on 8 (Q4_K) or 16 banks.  W[0] and W[NF + 1] hold only
        // bytes outside the unit, which no field uses.
        // Both forms write sh first and then W[0], W[1], ..., W[NF + 1] in that
        // order: branches that end in stores to different members get them
        // merged into one store at a selected address, which keeps the struct
        // in scratch memory.  Each wide word passes whole through an empty
        // asm: with only its elements used, the compiler otherwise splits it
        // into dword reads.
        constexpr int UB = UnitFmt<QT>::BYTES;
        constexpr int A = UB % 16 == 0 && (UB / 16) % 2 == 1 ? 16 : UB % 8 == 0 && (UB / 8) % 2 == 1 ? 8 : 0;
        const uint8_t* o = unit_lds + ORG - 4;
        sh = (uint32_t)(reinterpret_cast<uintptr_t>(o) & 3);   // ORG & 3 for an A-aligned unit
        if constexpr (A != 0 && 4 * NF == UB) {
            if ((reinterpret_cast<uintptr_t>(unit_lds) & (A - 1)) == 0) {
                typedef unsigned int v4u __attribute__((ext_vector_type(4)));
                typedef unsigned int v2u __attribute__((ext_vector_type(2)));
                W[0] = 0;
                if constexpr (A == 16) {
                    const v4u* g = reinterpret_cast<const v4u*>(unit_lds);
#pragma unroll
                    for (int c = 0; c < NF / 4; ++c) {
                        v4u v = g[c];
                        asm("" : "+v"(v));
                        W[1 + 4 * c] = v.x;
                        W[2 + 4 * c] = v.y;
                        W[3 + 4 * c] = v.z;
                        W[4 + 4 * c] = v.w;
                    }
                } else {
                    const v2u* g = reinterpret_cast<const v2u*>(unit_lds);
#pragma unroll
                    for (int c = 0; c < NF / 2; ++c) {
                        v2u v = g[c];
                        asm("" : "+v"(v));
                        W[1 + 2 * c] = v.x;
                        W[2 + 2 * c] = v.y;
                    }
                }
                W[NF + 1] = 0;
                return;
            }
        }
        const uint32_t* g = reinterpret_cast<const uint32_t*>(o - sh);
#pragma unroll
        for (int i = 0; i < NF + 2; ++i) W[i] = g[i];
    }
    __device__ inline void fields(uint32_t (&F)[NF], uint32_t& Fm1) const {
        Fm1 = __builtin_amdgcn_alignbyte(W[1], W[0], sh);
#pragma unroll
        for (int i = 0; i < NF; ++i) F[i] = __builtin_amdgcn_alignbyte(W[i + 2], W[i + 1], sh);
    }
};

__device__ inline float h2f(uint32_t bits16) { return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xFFFFu))); }

__device__ inline int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// ---------------------------------------------------------------------------
// LDS table for IQ3_S: the 512-entry codebook (u32: four magnitudes, one per
// byte) with every sign pattern already applied.  Entry qs + 256 * h, where
// h = n + 16 * b for a sign nibble n and ninth index bit b, holds
// grid[qs + 256 * b] with byte j negated where bit j of n is set; 8192 u32 at
// LDS byte 0.  A lookup's byte address is the 16-bit value [qs, h] times 4,
// and one v_perm builds that value for two lookups at once.
// ---------------------------------------------------------------------------
constexpr int kLdsGrid = 0;
constexpr int kLdsTables = 8192 * 4;

__device__ inline uint32_t spread4(uint32_t n) { return (n * 0x00204081u) & 0x01010101u; }

// (w & 0xFFFF) << 2, the byte address of the table index in w's low half, in
// one instruction: the SDWA operand select reads the low 16 bits of w (the
// compiler otherwise shifts and masks in two)
__device__ inline uint32_t lo16_x4(uint32_t w) {
    uint32_t a;
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
        : "=v"(a)
        : "v"(w));
    return a;
}

// v_perm selector that negates byte j of a codebook word g where bit j of n
// is set, taking that byte from g ^ 0xFEFEFEFE (source 0) instead of g
// (source 1): for odd g, -g = g ^ 0xFE (two's complement ~(g - 1), and
// g - 1 = g ^ 1).  n * 0x810204 puts bit j of n at bit 8j + 2 (the partial
// products do not overlap for n < 16), turning selector byte j into j + 4.
__host__ __device__ constexpr uint32_t sign_sel(uint32_t n) { return ((n * 0x00810204u) & 0x04040404u) | 0x03020100u; }

// The signed codebook in LDS, written by NT threads (w = 0 .. NT-1 of them)
// from codebook registers loaded early.
template <int NT>
struct GridRegs {
    static constexpr int N = NT >= 512 ? 1 : 512 / NT;   // entries per thread (threads 512.. hold none)
    uint32_t e[N];
};
template <int NT>
__device__ inline GridRegs<NT> load_grid_regs(int w) {
    GridRegs<NT> g;
#pragma unroll
    for (int i = 0; i < GridRegs<NT>::N; ++i) g.e[i] = kIq3sGridDev.e[min(w + NT * i, 511)];
    return g;
}
template <int NT>
__device__ inline void store_iq3s_tables(uint8_t* smem, const GridRegs<NT>& g, int w) {
    uint32_t* tab = reinterpret_cast<uint32_t*>(smem + kLdsGrid);
    if (NT > 512 && w >= 512) return;
#pragma unroll
    for (int i = 0; i < GridRegs<NT>::N; ++i) {
        const int idx = w + NT * i;                       // codebook index qs + 256 * b
        uint32_t* row = tab + (idx & 255) + 4096 * (idx >> 8);
        const uint32_t neg = g.e[i] ^ 0xFEFEFEFEu;
#pragma unroll
        for (int n = 0; n < 16; ++n) row[256 * n] = __builtin_amdgcn_perm(neg, g.e[i], sign_sel((uint32_t)n));
    }
}
// all 256 threads of the workgroup
__device__ inline void stage_iq3s_tables(uint8_t* smem) {
    store_iq3s_tables<256>(smem, load_grid_regs<256>((int)threadIdx.x), (int)threadIdx.x);
}

// IQ3_XXS: the 256-entry codebook with every sign pattern applied, 4096 u32
// at LDS byte 0: entry q + 256 * n holds grid[q] with byte j negated where bit
// j of the sign nibble n is set.  The magnitudes are even (4 .. 62), so a
// byte's negation is ~g + 1 (no carry leaves a byte).
constexpr int kLdsTablesXxs = 4096 * 4;

__device__ inline uint32_t neg_bytes(uint32_t g) { return ~g + 0x01010101u; }

// IQ2_S: the 1024-entry codebook unsigned, two dwords per entry (8 KB at LDS
// byte 0): one 8-byte read per eight weights, the signs applied in VALU.
constexpr int kLdsTablesIq2s = 2048 * 4;

// LDS table bytes of a weight type's decoder
__host__ __device__ constexpr int table_bytes(int qt) {
    return qt == QT_IQ3_S ? kLdsTables : qt == QT_IQ3_XXS ? kLdsTablesXxs : qt == QT_IQ2_S ? kLdsTablesIq2s : 0;
}

// Codebook words a thread loads early (the first NT threads of 512 / 256
// entries) and later expands into the LDS table; nothing for types without
// a table.
template <int QT, int NT>
struct TableRegs {
    static constexpr int ENTRIES = QT == QT_IQ3_S ? 512 : QT == QT_IQ3_XXS ? 256 : QT == QT_IQ2_S ? 2048 : 0;   // words
    static constexpr int N = ENTRIES == 0 ? 0 : (NT >= ENTRIES ? 1 : ENTRIES / NT);
    uint32_t e[N > 0 ? N : 1];
};
template <int QT, int NT>
__device__ inline TableRegs<QT, NT> load_tables(int w) {
    TableRegs<QT, NT> g;
    constexpr int E = TableRegs<QT, NT>::ENTRIES;
#pragma unroll
    for (int i = 0; i < TableRegs<QT, NT>::N; ++i) {
        const int idx = min(w + NT * i, E - 1);
        g.e[i] = QT == QT_IQ3_S ? kIq3sGridDev.e[idx] : QT == QT_IQ3_XXS ? kIq3xxsGridDev.e[idx] : kIq2sGridDev.w[idx];
    }
    return g;
}
template <int QT, int NT>
__device__ inline void store_tables(uint8_t* smem, const TableRegs<QT, NT>& g, int w) {
    if constexpr (QT == QT_IQ3_S) {
        GridRegs<NT> gr;
#pragma unroll
        for (int i = 0; i < GridRegs<NT>::N; ++i) gr.e[i] = g.e[i];
        store_iq3s_tables<NT>(smem, gr, w);
    } else if constexpr (QT == QT_IQ3_XXS) {
        uint32_t* tab = reinterpret_cast<uint32_t*>(smem + kLdsGrid);
        if (NT > 256 && w >= 256) return;
#pragma unroll
        for (int i = 0; i < TableRegs<QT, NT>::N; ++i) {
            const int idx = w + NT * i;
            const uint32_t neg = neg_bytes(g.e[i]);
#pragma unroll
            for (int n = 0; n < 16; ++n) tab[idx + 256 * n] = __builtin_amdgcn_perm(neg, g.e[i], sign_sel((uint32_t)n));
        }
    } else if constexpr (QT == QT_IQ2_S) {
        uint32_t* tab = reinterpret_cast<uint32_t*>(smem + kLdsGrid);
        if (NT > 2048 && w >= 2048) return;
#pragma unroll
        for (int i = 0; i < TableRegs<QT, NT>::N; ++i) tab[w + NT * i] = g.e[i];
    }
}

// IQ4_NL / IQ4_XS: the int8 levels of four 4-bit indices (one per byte):
// two v_perm over the 16 levels (low eight, high eight) and a per-byte
// select on bit 3 of the index.
__device__ inline uint32_t iq4_levels(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4nlLevelWords[1], kIq4nlLevelWords[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4nlLevelWords[3], kIq4nlLevelWords[2], sel);
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, 0x0C0C0C0Cu | ((n >> 3) & 0x01010101u));   // 0xFF where bit 3 set
    return (hi & m) | (lo & ~m);
}

__device__ inline uint32_t lds_u32(const uint8_t* smem, uint32_t byte_off) {
    return *reinterpret_cast<const uint32_t*>(smem + byte_off);
}

// 32 activation bytes of item j of a 256-element chunk (8 dwords)
__device__ inline void act8(const uint8_t* chunk, int j, uint32_t (&A)[8]) {
    const uint4 a0 = reinterpret_cast<const uint4*>(chunk)[2 * j];
    const uint4 a1 = reinterpret_cast<const uint4*>(chunk)[2 * j + 1];
    A[0] = a0.x; A[1] = a0.y; A[2] = a0.z; A[3] = a0.w;
    A[4] = a1.x; A[5] = a1.y; A[6] = a1.z; A[7] = a1.w;
}

// ---------------------------------------------------------------------------
// IQ3_S: element 32*ib + 4*g + j = ls(ib) * grid[qs[8ib+g] | bit g of qh[ib] << 8][j]
//        * (-1 if bit (4*(g&1)+j) of signs[4ib + g/2]); ls = 2*scale_nibble + 1.
// F[0..15] qs, F[16..17] qh, F[18..25] signs, F[26] scales, Fm1 >> 16 = d.
// ---------------------------------------------------------------------------
// packed int8 weights of item ib (8 dwords) and its scale
__device__ inline int iq3s_item(const uint32_t (&F)[27], int ib, const uint8_t* smem, uint32_t (&v)[8]) {
    const uint32_t qh = (F[16 + (ib >> 2)] >> (8 * (ib & 3))) & 0xFFu;
    const uint32_t S = F[18 + ib];           // sign nibble of grid g at bits 4g..4g+3
    // H[k] byte j: h of grid g = 4k + j (its sign nibble | bit g of qh << 4)
    uint32_t H[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t x = __builtin_amdgcn_perm(S, S, k ? 0x0C030C02u : 0x0C010C00u);   // [S.b2k, 0, S.b2k+1, 0]
        const uint32_t y = (x | (x << 4)) & 0x0F0F0F0Fu;                                 // one nibble per byte
        // bit j of the qh nibble to bit 8j + 4 (a 24-bit multiply: the shift is not folded into a 32-bit one)
        H[k] = y | (__umul24(k ? qh & 0xF0u : (qh & 15u) << 4, 0x00204081u) & 0x10101010u);
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t Q = F[2 * ib + (l >> 1)];
        const uint32_t pp = 2u * (uint32_t)(l & 1);
        // [qs_g, h_g, qs_g+1, h_g+1] for g = 2l: two 16-bit table indices
        const uint32_t sel = (4u + pp) | (pp << 8) | ((5u + pp) << 16) | ((pp + 1u) << 24);
        const uint32_t D = __builtin_amdgcn_perm(Q, H[l >> 1], sel);
        v[2 * l] = lds_u32(smem, kLdsGrid + lo16_x4(D));
        v[2 * l + 1] = lds_u32(smem, kLdsGrid + (D >> 14));      // h < 32: bits 14, 15 of D are 0
    }
    return 2 * (int)((F[26] >> (4 * ib)) & 15u) + 1;
}

// Half h (items 4h .. 4h + 3, h = 0 or 1 per lane) of an IQ3_S unit staged in
// LDS at byte address unit_lds, read straight into the places iq3s_item
// reads for items 0..3: G[0..7] the half's 32 qs bytes, G[16] its qh bytes,
// G[18..21] its sign bytes, G[26] (low 16 bits) its scale nibbles.  The
// unit's fp16 d is returned in the low 16 bits of dbits.  A unit starts at an
// even byte, so every field is one byte shift (0 or 2) away from the dword
// grid: 20 dword reads instead of the unit's 29.  Bytes outside the unit
// (the two before it) are read but never used.
__device__ inline void iq3s_half_fields(const uint8_t* unit_lds, int h, uint32_t (&G)[27], uint32_t& dbits) {
    const uint8_t* o = unit_lds + 2;                                 // qs; qh at +64, signs +72, scales +104
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(o) & 3);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(o - sh);
    const uint32_t* qq = q + 8 * h;                                   // the half's qs
    uint32_t W[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) W[i] = qq[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) G[i] = __builtin_amdgcn_alignbyte(W[i + 1], W[i], sh);
    const uint32_t* qh = q + 16 + h;
    G[16] = __builtin_amdgcn_alignbyte(qh[1], qh[0], sh);
    const uint32_t* sg = q + 18 + 4 * h;
    uint32_t S[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) S[i] = sg[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) G[18 + i] = __builtin_amdgcn_alignbyte(S[i + 1], S[i], sh);
    G[26] = __builtin_amdgcn_alignbyte(q[27], q[26], sh) >> (16 * h);
    dbits = __builtin_amdgcn_alignbyte(q[0], q[-1], sh) >> 16;
}

// the 128 activation bytes of half h of a 256-element chunk, per item
__device__ inline void act_half(const uint8_t* chunk, int h, uint32_t (&A)[4][8]) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) act8(chunk + 128 * h, ib, A[ib]);
}

// The exact integer sum over the four items of a half (iq3s_half_fields):
// sum ls(ib) * (weights . activations).
__device__ inline int iq3s_half_bsum(const uint32_t (&G)[27], const uint8_t* smem, const uint32_t (&A)[4][8]) {
    int bsum = 0;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
        uint32_t v[8];
        const int ls = iq3s_item(G, ib, smem, v);
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[ib][i], s);
        bsum += __mul24(ls, s);
    }
    return bsum;
}

// The same sum in two steps: the weights of the half decoded to int8 first
// (no activations needed), dotted with them later.  The integer sum is the
// same as iq3s_half_bsum's.
struct Iq3sHalf {
    uint32_t v[4][8];       // int8 weights of items 0..3 of the half
    int ls[4];              // their scales 2 * nibble + 1
};
__device__ inline void iq3s_half_decode(const uint32_t (&G)[27], const uint8_t* smem, Iq3sHalf& W) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) W.ls[ib] = iq3s_item(G, ib, smem, W.v[ib]);
}
__device__ inline int iq3s_half_dot(const Iq3sHalf& W, const uint32_t (&A)[4][8]) {
    int bsum = 0;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(W.v[ib][i], A[ib][i], s);
        bsum += __mul24(W.ls[ib], s);
    }
    return bsum;
}

// ---------------------------------------------------------------------------
// Q4_K: element 32j + l = d*sc_j*nib - dmin*m_j, nibble low (j even) / high (j
// odd) of qs[32*(j/2) + l].  F[0] = d | dmin << 16, F[1..3] packed 6-bit
// scales/mins (get_scale_min_k4), F[4..35] qs.
// ---------------------------------------------------------------------------
__device__ inline uint32_t byte_of(const uint32_t* F, int b) { return (F[b >> 2] >> (8 * (b & 3))) & 0xFFu; }

template <int NF>
__device__ inline void q4k_scale_min(const uint32_t (&F)[NF], int j, int& sc, int& mn) {
    const uint32_t* q = F + 1;      // the 12 scale bytes
    if (j < 4) {
        sc = (int)(byte_of(q, j) & 63u);
        mn = (int)(byte_of(q, j + 4) & 63u);
    } else {
        sc = (int)((byte_of(q, j + 4) & 0xFu) | ((byte_of(q, j - 4) >> 6) << 4));
        mn = (int)((byte_of(q, j + 4) >> 4) | ((byte_of(q, j) >> 6) << 4));
    }
}

__device__ inline void q4k_item(const uint32_t (&F)[36], int j, uint32_t (&v)[8]) {
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (F[4 + 8 * (j >> 1) + i] >> sh) & 0x0F0F0F0Fu;
}

// Half h of a Q4_K unit staged in LDS (items 4h .. 4h + 3, two lanes per
// unit): F[0..3] the unit's d, dmin and packed scales / mins, F[4..19] its qs
// bytes 64h .. 64h + 63 (so item 4h + j takes F[4 + 8 (j / 2) ..]).  A
// 16-byte aligned unit is read as five 16-byte words, otherwise as dwords
// shifted into place.
struct Q4kHalf {
    uint32_t F[20];
};
__device__ inline void q4k_half_fields(const uint8_t* unit_lds, int h, Q4kHalf& Q) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    if ((reinterpret_cast<uintptr_t>(unit_lds) & 15) == 0) {
        const v4u* g = reinterpret_cast<const v4u*>(unit_lds);
#pragma unroll
        for (int c = 0; c < 5; ++c) {
            v4u v = g[c == 0 ? 0 : 4 * h + c];
            asm("" : "+v"(v));
            Q.F[4 * c] = v.x; Q.F[4 * c + 1] = v.y; Q.F[4 * c + 2] = v.z; Q.F[4 * c + 3] = v.w;
        }
        return;
    }
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(unit_lds) & 3);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(unit_lds - sh);
    uint32_t W[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) W[i] = w[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) Q.F[i] = __builtin_amdgcn_alignbyte(W[i + 1], W[i], sh);
    const uint32_t* wq = w + 4 + 16 * h;
    uint32_t V[17];
#pragma unroll
    for (int i = 0; i < 17; ++i) V[i] = wq[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) Q.F[4 + i] = __builtin_amdgcn_alignbyte(V[i + 1], V[i], sh);
}
// The exact integer sums of a half against the q8_K chunk's items (activation
// bytes A of items 4h .. 4h + 3, bsums bs of the whole chunk):
// isum = sum sc_j (q_j . x_j), msum = sum mn_j (bsum_2j + bsum_2j+1).
__device__ inline void q4k_half_sums(const Q4kHalf& Q, int h, const uint32_t (&A)[4][8], const int16_t* bs, int& isum,
                                     int& msum) {
    isum = 0;
    msum = 0;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int j = 4 * h + jj;
        const int sh = 4 * (jj & 1);
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4((Q.F[4 + 8 * (jj >> 1) + i] >> sh) & 0x0F0F0F0Fu, A[jj][i], s);
        int sc, mn;
        q4k_scale_min(Q.F, j, sc, mn);
        isum += __mul24(sc, s);
        msum += __mul24(mn, (int)bs[2 * j] + (int)bs[2 * j + 1]);
    }
}

// ---------------------------------------------------------------------------
// Q5_K: Q4_K's d, dmin and packed 6-bit scales / mins in F[0..3], qh[32] in
// F[4..11], qs[128] in F[12..43]; element 32 j + l (sub-block j) is the nibble
// (low for even j) of qs[32 (j / 2) + l] plus 16 when bit j of qh[l] is set.
// ---------------------------------------------------------------------------
__device__ inline void q5k_item(const uint32_t (&F)[44], int j, uint32_t (&v)[8]) {
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = ((F[12 + 8 * (j >> 1) + i] >> sh) & 0x0F0F0F0Fu) | (((F[4 + i] >> j) & 0x01010101u) << 4);
}

// ---------------------------------------------------------------------------
// Q5_1 (four 24-byte blocks per unit): block J's fp16 d and m in F[6 J], qh in
// F[6 J + 1], qs in F[6 J + 2 .. 6 J + 5]; element j < 16 is the low nibble of
// qs[j] plus bit j of qh times 16, element j + 16 the high nibble plus bit
// j + 16; value d q + m.  v: the 32 values as int8 (0 .. 31) in element order.
// ---------------------------------------------------------------------------
__device__ inline uint32_t spread4_x16(uint32_t n) { return spread4(n) << 4; }
template <int J>
__device__ inline void q5_1_block(const uint32_t (&F)[24], uint32_t (&v)[8], uint32_t& dm) {
    dm = F[6 * J];
    const uint32_t qh = F[6 * J + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = F[6 * J + 2 + i];
        v[i] = (q & 0x0F0F0F0Fu) | spread4_x16((qh >> (4 * i)) & 15u);
        v[4 + i] = ((q >> 4) & 0x0F0F0F0Fu) | spread4_x16((qh >> (16 + 4 * i)) & 15u);
    }
}

// ---------------------------------------------------------------------------
// Q6_K: item j (elements 32j..32j+31) = half h = j/4, quarter q = j%4: low 4 bits
// from ql[64h + 32(q&1) + l] (nibble q>>1), high 2 bits from qh[32h + l] bits 2q..;
// value (q6 - 32) * d * sc[16-element half].  F[0..31] ql, F[32..47] qh,
// F[48..51] int8 scales, F[52] & 0xFFFF = d.
// ---------------------------------------------------------------------------
__device__ inline void q6k_item(const uint32_t (&F)[53], int j, uint32_t (&v)[8]) {
    const int h = j >> 2, q = j & 3;
    const int nsh = 4 * (q >> 1), hsh = 2 * q;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = ((F[16 * h + 8 * (q & 1) + i] >> nsh) & 0x0F0F0F0Fu) | (((F[32 + 8 * h + i] >> hsh) & 0x03030303u) << 4);
}
__device__ inline int q6k_scale(const uint32_t (&F)[53], int s16) {
    return (int)(int8_t)((F[48 + (s16 >> 2)] >> (8 * (s16 & 3))) & 0xFFu);
}

// ---------------------------------------------------------------------------
// Q8_0 unit = 4 blocks of 34 B; block j at unit byte 34j: d at 34j, qs at 34j+2.
// With the field origin at unit byte 2, block j's d is at F-byte 34j-2 and its
// qs at F-byte 34j (dword aligned for even j, 2 past a dword for odd j).
// ---------------------------------------------------------------------------
template <int J>
__device__ inline void q8_0_block(const uint32_t (&F)[34], uint32_t Fm1, uint32_t (&v)[8], uint32_t& dbits) {
    constexpr int qo = 34 * J;               // F-byte of the qs
    if constexpr ((qo & 3) == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = F[qo / 4 + i];
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_amdgcn_alignbyte(F[qo / 4 + i + 1], F[qo / 4 + i], 2);
    }
    constexpr int dob = qo - 2;              // F-byte of d (even)
    if constexpr (dob < 0) dbits = Fm1 >> 16;
    else if constexpr ((dob & 3) == 0) dbits = F[dob / 4] & 0xFFFFu;
    else dbits = F[dob / 4] >> 16;
}

// ---------------------------------------------------------------------------
// IQ3_XXS: element 32 ib + 8 l + 4 h + j = ls(ib) * grid[qs[8 ib + 2 l + h]][j]
//        * (-1 if bit 4 h + j of ksigns[(aux >> 7 l) & 127]), aux = the u32
// of sub-block ib, ls = 2 * (aux >> 28) + 1 (the 0.5 + nibble of ggml, times
// two: the result carries a final factor 0.25).  ksigns[i] is i with an
// even-parity bit 7.  F[0..15] qs, F[16..23] aux, Fm1 >> 16 = d.
// ---------------------------------------------------------------------------
__device__ inline int iq3xxs_item(const uint32_t (&F)[24], int ib, const uint8_t* smem, uint32_t (&v)[8]) {
    const uint32_t aux = F[16 + ib];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
        const uint32_t sg = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
        const uint32_t q2 = (F[2 * ib + (l >> 1)] >> (16 * (l & 1))) & 0xFFFFu;   // grid indices of 8 l, 8 l + 4
        v[2 * l] = lds_u32(smem, kLdsGrid + 4u * ((q2 & 0xFFu) | ((sg & 15u) << 8)));
        v[2 * l + 1] = lds_u32(smem, kLdsGrid + 4u * ((q2 >> 8) | ((sg >> 4) << 8)));
    }
    return 2 * (int)(aux >> 28) + 1;
}

// ---------------------------------------------------------------------------
// IQ2_S: element 32 ib + 8 l + j = db(l) * grid[qs[4 ib + l] | qh bits 2l,
// 2l+1 << 8][j] * (-1 if bit j of signs[4 ib + l]); ls = 2 * nibble + 1, the
// low nibble of scales[ib] for l < 2, the high one after (ggml's result
// carries a final factor 0.125).  F[0..7] qs, F[8..15] signs, F[16..17] qh,
// F[18..19] scales, Fm1 >> 16 = d.  The magnitudes (8, 25, 43) are negated
// byte-wise as ~g + 1.
// ---------------------------------------------------------------------------
__device__ inline void iq2s_group(const uint32_t (&F)[20], int ib, int l, const uint8_t* smem, uint32_t& lo,
                                  uint32_t& hi) {
    const uint32_t qh = byte_of(F + 16, ib);
    const uint32_t gi = byte_of(F, 4 * ib + l) | (((qh >> (2 * l)) & 3u) << 8);
    const uint2 g = *reinterpret_cast<const uint2*>(smem + kLdsGrid + 8u * gi);
    const uint32_t sg = byte_of(F + 8, 4 * ib + l);
    lo = __builtin_amdgcn_perm(neg_bytes(g.x), g.x, sign_sel(sg & 15u));
    hi = __builtin_amdgcn_perm(neg_bytes(g.y), g.y, sign_sel(sg >> 4));
}

// ---------------------------------------------------------------------------
// IQ4_NL unit = 4 blocks of 18 B: d at 18 j, qs[16] at 18 j + 2; element
// 32 j + i = d * kvalues[qs[i] & 15], element 32 j + 16 + i = d *
// kvalues[qs[i] >> 4].  With the origin at unit byte 2, block j's qs sit at
// F-byte 18 j (dword aligned for even j) and its d at F-byte 18 j - 2.
// ---------------------------------------------------------------------------
template <int J>
__device__ inline void iq4nl_block(const uint32_t (&F)[18], uint32_t Fm1, uint32_t (&qd)[4], uint32_t& dbits) {
    constexpr int qo = 18 * J;
    if constexpr ((qo & 3) == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) qd[i] = F[qo / 4 + i];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) qd[i] = __builtin_amdgcn_alignbyte(F[qo / 4 + i + 1], F[qo / 4 + i], 2);
    }
    constexpr int dob = qo - 2;
    if constexpr (dob < 0) dbits = Fm1 >> 16;
    else if constexpr ((dob & 3) == 0) dbits = F[dob / 4] & 0xFFFFu;
    else dbits = F[dob / 4] >> 16;
}

// ---------------------------------------------------------------------------
// Q2_0 unit = 4 blocks of 18 B, 64 elements each: the byte layout of an IQ4_NL
// unit, so block J's d and 16 code bytes come out of iq4nl_block<J>.  Code e
// of a block sits at bits 2*(e % 4) of byte e / 4; its value is (code - 1) * d
// (sabah_rt.cu:2411-2419).
// ---------------------------------------------------------------------------
// code - 1 as int8, for the codes in the low two bits of each byte of x
__device__ inline uint32_t q2_0_values(uint32_t x) {
    return __builtin_amdgcn_perm(0u, 0x020100FFu, x & 0x03030303u);   // selector 0..3 -> -1, 0, 1, 2
}
// the 16 codes of code dword w as int8 values in element order: o[g] byte i is
// element 4g + i (bits 2i of byte g)
__device__ inline void q2_0_dword(uint32_t w, uint32_t (&o)[4]) {
    const uint32_t c0 = q2_0_values(w), c1 = q2_0_values(w >> 2), c2 = q2_0_values(w >> 4),
                   c3 = q2_0_values(w >> 6);
    // 4 x 4 byte transpose: byte g of c_i becomes byte i of o[g]
    const uint32_t p0 = __builtin_amdgcn_perm(c1, c0, 0x05010400u);   // c0.b0 c1.b0 c0.b1 c1.b1
    const uint32_t p1 = __builtin_amdgcn_perm(c1, c0, 0x07030602u);   // c0.b2 c1.b2 c0.b3 c1.b3
    const uint32_t p2 = __builtin_amdgcn_perm(c3, c2, 0x05010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(c3, c2, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(p2, p0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(p2, p0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(p3, p1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(p3, p1, 0x07060302u);
}
// the integer dot of 32 codes (two code dwords) with 32 activations
__device__ inline int q2_0_dot32(const uint32_t* qd, const uint32_t* A) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t o[4];
        q2_0_dword(qd[i], o);
#pragma unroll
        for (int g = 0; g < 4; ++g) s = sdot4(o[g], A[4 * i + g], s);
    }
    return s;
}

// the integer dot of 16 level bytes (four dwords of nibble pairs) with 32
// activations: low nibbles against A[0..3], high nibbles against A[4..7]
__device__ inline int iq4_dot32(const uint32_t* qd, const uint32_t* A) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = sdot4(iq4_levels(qd[i] & 0x0F0F0F0Fu), A[i], s);
#pragma unroll
    for (int i = 0; i < 4; ++i) s = sdot4(iq4_levels((qd[i] >> 4) & 0x0F0F0F0Fu), A[4 + i], s);
    return s;
}

// ---------------------------------------------------------------------------
// unit dot: contribution(s) of one unit to its row, ggml's float order per
// block: (d_w * d_x) * isum  [Q4_K: minus (dmin_w * d_x) * msum]
//   chunk: LDS activation bytes of the unit's 256-element chunk
//   dx   : activation scale(s) of the unit's block(s); bs: its q8_K bsums
// ---------------------------------------------------------------------------
template <int QT>
struct UnitDot {
    float c[UnitFmt<QT>::CONTRIB];
};

template <int QT, typename Window>
__device__ inline UnitDot<QT> unit_dot(const Window& Wn, const uint8_t* smem, const uint8_t* chunk,
                                       const float* dx, const int16_t* bs) {
    uint32_t F[UnitFmt<QT>::NF];
    uint32_t Fm1;
    Wn.fields(F, Fm1);
    UnitDot<QT> r;
    if constexpr (QT == QT_IQ3_S) {
        int bsum = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t v[8], A[8];
            const int ls = iq3s_item(F, ib, smem, v);
            act8(chunk, ib, A);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s);
            bsum += __mul24(ls, s);              // |s| <= 32 * 15 * 127 < 2^23
        }
        r.c[0] = __fmul_rn(__fmul_rn(h2f(Fm1 >> 16), dx[0]), (float)bsum);
    } else if constexpr (QT == QT_Q4_K) {
        int isum = 0, msum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8], A[8];
            q4k_item(F, j, v);
            act8(chunk, j, A);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s);
            int sc, mn;
            q4k_scale_min(F, j, sc, mn);
            isum += __mul24(sc, s);             // sc, mn < 64; |s| < 2^16
            msum += __mul24(mn, (int)bs[2 * j] + (int)bs[2 * j + 1]);
        }
        const float d = h2f(F[0]), dmin = h2f(F[0] >> 16);
        r.c[0] = __fsub_rn(__fmul_rn(__fmul_rn(d, dx[0]), (float)isum), __fmul_rn(__fmul_rn(dmin, dx[0]), (float)msum));
    } else if constexpr (QT == QT_Q5_K) {
        int isum = 0, msum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8], A[8];
            q5k_item(F, j, v);
            act8(chunk, j, A);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s);
            int sc, mn;
            q4k_scale_min(F, j, sc, mn);
            isum += __mul24(sc, s);             // sc, mn < 64; |s| < 2^17
            msum += __mul24(mn, (int)bs[2 * j] + (int)bs[2 * j + 1]);
        }
        const float d = h2f(F[0]), dmin = h2f(F[0] >> 16);
        r.c[0] = __fsub_rn(__fmul_rn(__fmul_rn(d, dx[0]), (float)isum), __fmul_rn(__fmul_rn(dmin, dx[0]), (float)msum));
    } else if constexpr (QT == QT_Q5_1) {
        // ggml: per block sumf += (d_w * d_x) * sumi + m_w * s_x; bs carries the q8_1 s values
        const float* sx = reinterpret_cast<const float*>(bs);
        uint32_t v[8], A[8], dm;
#define SB_Q51_BLOCK(J)                                                                          \
        {                                                                                        \
            q5_1_block<J>(F, v, dm);                                                             \
            act8(chunk, J, A);                                                                   \
            int s = 0;                                                                           \
            _Pragma("unroll") for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s);              \
            r.c[J] = __fadd_rn(__fmul_rn(__fmul_rn(h2f(dm), dx[J]), (float)s), __fmul_rn(h2f(dm >> 16), sx[J])); \
        }
        SB_Q51_BLOCK(0) SB_Q51_BLOCK(1) SB_Q51_BLOCK(2) SB_Q51_BLOCK(3)
#undef SB_Q51_BLOCK
    } else if constexpr (QT == QT_Q6_K) {
        int isum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8], A[8];
            q6k_item(F, j, v);
            act8(chunk, j, A);
            int sa = 0, sb = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) sa = sdot4(v[i], A[i], sa);
#pragma unroll
            for (int i = 4; i < 8; ++i) sb = sdot4(v[i], A[i], sb);
            // sum (q - 32) * q8 = sum q * q8 - 32 * bsum over each 16-element half
            sa -= 32 * (int)bs[2 * j];
            sb -= 32 * (int)bs[2 * j + 1];
            isum += __mul24(q6k_scale(F, 2 * j), sa) + __mul24(q6k_scale(F, 2 * j + 1), sb);   // |sa|, |sb| < 2^18
        }
        r.c[0] = __fmul_rn(__fmul_rn(h2f(F[52]), dx[0]), (float)isum);
    } else if constexpr (QT == QT_IQ3_XXS) {
        // ggml: sumf += (d_w * d_x) * bsum per super-block, result 0.25 * sumf;
        // the power-of-two factor is applied per contribution (exact)
        int bsum = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t v[8], A[8];
            const int ls = iq3xxs_item(F, ib, smem, v);
            act8(chunk, ib, A);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s);
            bsum += __mul24(ls, s);              // |s| <= 32 * 62 * 127 < 2^18
        }
        r.c[0] = __fmul_rn(__fmul_rn(__fmul_rn(h2f(Fm1 >> 16), dx[0]), (float)bsum), 0.25f);
    } else if constexpr (QT == QT_IQ2_S) {
        // ggml: sumf += (d_w * d_x) * bsum per super-block, result 0.125 * sumf;
        // the power-of-two factor is applied per contribution (exact)
        int bsum = 0;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t A[8];
            act8(chunk, ib, A);
            int s[2] = {0, 0};
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                uint32_t lo, hi;
                iq2s_group(F, ib, l, smem, lo, hi);
                s[l >> 1] = sdot4(hi, A[2 * l + 1], sdot4(lo, A[2 * l], s[l >> 1]));
            }
            const uint32_t sc = byte_of(F + 18, ib);
            bsum += __mul24(2 * (int)(sc & 15u) + 1, s[0]) + __mul24(2 * (int)(sc >> 4) + 1, s[1]);   // |s| < 2^15
        }
        r.c[0] = __fmul_rn(__fmul_rn(__fmul_rn(h2f(Fm1 >> 16), dx[0]), (float)bsum), 0.125f);
    } else if constexpr (QT == QT_IQ4_XS) {
        // ggml: per 32-element sub-block sumf += ((d_w * d_x) * (ls - 32)) * sumi
        const float d4d8 = __fmul_rn(h2f(F[0]), dx[0]);
        const uint32_t sh = F[0] >> 16;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t A[8];
            act8(chunk, ib, A);
            const int s = iq4_dot32(F + 2 + 4 * ib, A);
            const int ls = (int)((F[1] >> (4 * ib)) & 15u) | (int)(((sh >> (2 * ib)) & 3u) << 4);
            r.c[ib] = __fmul_rn(__fmul_rn(d4d8, (float)(ls - 32)), (float)s);
        }
    } else if constexpr (QT == QT_IQ4_NL) {   // four independent q8_0-paired blocks
        uint32_t qd[4], A[8], db;
#define SB_IQ4NL_BLOCK(J)                                                                  \
        {                                                                                  \
            iq4nl_block<J>(F, Fm1, qd, db);                                                \
            act8(chunk, J, A);                                                             \
            r.c[J] = __fmul_rn(__fmul_rn(dx[J], h2f(db)), (float)iq4_dot32(qd, A));       \
        }
        SB_IQ4NL_BLOCK(0) SB_IQ4NL_BLOCK(1) SB_IQ4NL_BLOCK(2) SB_IQ4NL_BLOCK(3)
#undef SB_IQ4NL_BLOCK
    } else if constexpr (QT == QT_Q2_0) {    // four blocks, each paired with two q8_0 blocks
        uint32_t qd[4], A[8], db;
#define SB_Q20_BLOCK(J)                                                                    \
        {                                                                                  \
            iq4nl_block<J>(F, Fm1, qd, db);                                                \
            const float dw = h2f(db);                                                      \
            act8(chunk, 2 * J, A);                                                         \
            r.c[2 * J] = __fmul_rn((float)q2_0_dot32(qd, A), __fmul_rn(dw, dx[2 * J]));   \
            act8(chunk, 2 * J + 1, A);                                                     \
            r.c[2 * J + 1] = __fmul_rn((float)q2_0_dot32(qd + 2, A), __fmul_rn(dw, dx[2 * J + 1])); \
        }
        SB_Q20_BLOCK(0) SB_Q20_BLOCK(1) SB_Q20_BLOCK(2) SB_Q20_BLOCK(3)
#undef SB_Q20_BLOCK
    } else {   // Q8_0: four independent blocks
        uint32_t v[8], A[8], db;
#define SB_Q8_BLOCK(J)                                                              \
        {                                                                           \
            q8_0_block<J>(F, Fm1, v, db);                                           \
            act8(chunk, J, A);                                                      \
            int s = 0;                                                              \
            _Pragma("unroll") for (int i = 0; i < 8; ++i) s = sdot4(v[i], A[i], s); \
            r.c[J] = __fmul_rn((float)s, __fmul_rn(h2f(db), dx[J]));                \
        }
        SB_Q8_BLOCK(0) SB_Q8_BLOCK(1) SB_Q8_BLOCK(2) SB_Q8_BLOCK(3)
#undef SB_Q8_BLOCK
    }
    return r;
}

// ---------------------------------------------------------------------------
// dequantised values of a unit, ggml dequantize_row_* float order, through the
// same field extraction and item decoders as unit_dot
// ---------------------------------------------------------------------------
// n: elements of the unit to write (a row's last Q8_0 unit may be partial)
template <int QT>
__device__ inline void unit_dequant(const UnitWindow<QT>& Wn, const uint8_t* smem, float* out, int n) {
    uint32_t F[UnitFmt<QT>::NF];
    uint32_t Fm1;
    Wn.fields(F, Fm1);
    if constexpr (QT == QT_IQ3_S) {
        const float d = h2f(Fm1 >> 16);
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t v[8];
            const int ls = iq3s_item(F, ib, smem, v);
            const float db = __fmul_rn(d, (float)ls);           // d * (1 + 2*scale)
            for (int e = 0; e < 32; ++e)
                out[32 * ib + e] = __fmul_rn(db, (float)(int8_t)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu));
        }
    } else if constexpr (QT == QT_Q4_K) {
        const float d = h2f(F[0]), dmin = h2f(F[0] >> 16);
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8];
            q4k_item(F, j, v);
            int sc, mn;
            q4k_scale_min(F, j, sc, mn);
            const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
            for (int e = 0; e < 32; ++e)
                out[32 * j + e] = __fsub_rn(__fmul_rn(d1, (float)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu)), m1);
        }
    } else if constexpr (QT == QT_Q5_K) {
        const float d = h2f(F[0]), dmin = h2f(F[0] >> 16);
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8];
            q5k_item(F, j, v);
            int sc, mn;
            q4k_scale_min(F, j, sc, mn);
            const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
            for (int e = 0; e < 32; ++e)
                out[32 * j + e] = __fsub_rn(__fmul_rn(d1, (float)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu)), m1);
        }
    } else if constexpr (QT == QT_Q5_1) {
        uint32_t v[8], dm;
#define SB_Q51_DEQ(J)                                                                              \
        {                                                                                          \
            q5_1_block<J>(F, v, dm);                                                               \
            const float d = h2f(dm), m = h2f(dm >> 16);                                            \
            if (32 * J < n)                                                                        \
                for (int e = 0; e < 32; ++e)                                                       \
                    out[32 * J + e] = __fadd_rn(__fmul_rn((float)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu), d), m); \
        }
        SB_Q51_DEQ(0) SB_Q51_DEQ(1) SB_Q51_DEQ(2) SB_Q51_DEQ(3)
#undef SB_Q51_DEQ
    } else if constexpr (QT == QT_Q6_K) {
        const float d = h2f(F[52]);
        for (int j = 0; j < 8; ++j) {
            uint32_t v[8];
            q6k_item(F, j, v);
            for (int e = 0; e < 32; ++e) {
                const int q = (int)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu) - 32;
                out[32 * j + e] = __fmul_rn(__fmul_rn(d, (float)q6k_scale(F, 2 * j + (e >> 4))), (float)q);
            }
        }
    } else if constexpr (QT == QT_IQ3_XXS) {
        const float d = h2f(Fm1 >> 16);
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t v[8];
            iq3xxs_item(F, ib, smem, v);
            const float db = __fmul_rn(__fmul_rn(d, __fadd_rn(0.5f, (float)(F[16 + ib] >> 28))), 0.5f);
            for (int e = 0; e < 32; ++e)
                out[32 * ib + e] = __fmul_rn(db, (float)(int8_t)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu));
        }
    } else if constexpr (QT == QT_IQ2_S) {
        const float d = h2f(Fm1 >> 16);
        for (int ib = 0; ib < 8; ++ib) {
            const uint32_t sc = byte_of(F + 18, ib);
            const float db0 = __fmul_rn(__fmul_rn(d, __fadd_rn(0.5f, (float)(sc & 15u))), 0.25f);
            const float db1 = __fmul_rn(__fmul_rn(d, __fadd_rn(0.5f, (float)(sc >> 4))), 0.25f);
            for (int l = 0; l < 4; ++l) {
                uint32_t v[2];
                iq2s_group(F, ib, l, smem, v[0], v[1]);
                const float dl = l < 2 ? db0 : db1;
                for (int e = 0; e < 8; ++e)
                    out[32 * ib + 8 * l + e] = __fmul_rn(dl, (float)(int8_t)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu));
            }
        }
    } else if constexpr (QT == QT_IQ4_XS) {
        const float d = h2f(F[0]);
        const uint32_t sh = F[0] >> 16;
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = (int)((F[1] >> (4 * ib)) & 15u) | (int)(((sh >> (2 * ib)) & 3u) << 4);
            const float dl = __fmul_rn(d, (float)(ls - 32));
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = F[2 + 4 * ib + i];
                const uint32_t lo = iq4_levels(q & 0x0F0F0F0Fu), hi = iq4_levels((q >> 4) & 0x0F0F0F0Fu);
                for (int b = 0; b < 4; ++b) {
                    out[32 * ib + 4 * i + b] = __fmul_rn(dl, (float)(int8_t)((lo >> (8 * b)) & 0xFFu));
                    out[32 * ib + 16 + 4 * i + b] = __fmul_rn(dl, (float)(int8_t)((hi >> (8 * b)) & 0xFFu));
                }
            }
        }
    } else if constexpr (QT == QT_IQ4_NL) {
        uint32_t qd[4], db;
#define SB_IQ4NL_DEQ(J)                                                                              \
        {                                                                                            \
            iq4nl_block<J>(F, Fm1, qd, db);                                                          \
            const float d = h2f(db);                                                                 \
            if (32 * J < n)                                                                          \
                for (int i = 0; i < 4; ++i) {                                                        \
                    const uint32_t lo = iq4_levels(qd[i] & 0x0F0F0F0Fu);                             \
                    const uint32_t hi = iq4_levels((qd[i] >> 4) & 0x0F0F0F0Fu);                      \
                    for (int b = 0; b < 4; ++b) {                                                    \
                        out[32 * J + 4 * i + b] = __fmul_rn(d, (float)(int8_t)((lo >> (8 * b)) & 0xFFu));      \
                        out[32 * J + 16 + 4 * i + b] = __fmul_rn(d, (float)(int8_t)((hi >> (8 * b)) & 0xFFu)); \
                    }                                                                                \
                }                                                                                    \
        }
        SB_IQ4NL_DEQ(0) SB_IQ4NL_DEQ(1) SB_IQ4NL_DEQ(2) SB_IQ4NL_DEQ(3)
#undef SB_IQ4NL_DEQ
    } else if constexpr (QT == QT_Q2_0) {
        uint32_t qd[4], db;
#define SB_Q20_DEQ(J)                                                                               \
        {                                                                                           \
            iq4nl_block<J>(F, Fm1, qd, db);                                                         \
            const float d = h2f(db);                                                                \
            if (64 * J < n)                                                                         \
                for (int i = 0; i < 4; ++i) {                                                       \
                    uint32_t o[4];                                                                  \
                    q2_0_dword(qd[i], o);                                                           \
                    for (int e = 0; e < 16; ++e)                                                    \
                        out[64 * J + 16 * i + e] =                                                  \
                            __fmul_rn((float)(int8_t)((o[e >> 2] >> (8 * (e & 3))) & 0xFFu), d);    \
                }                                                                                   \
        }
        SB_Q20_DEQ(0) SB_Q20_DEQ(1) SB_Q20_DEQ(2) SB_Q20_DEQ(3)
#undef SB_Q20_DEQ
    } else {
        uint32_t v[8], db;
#define SB_Q8_DEQ(J)                                                                                       \
        {                                                                                                  \
            q8_0_block<J>(F, Fm1, v, db);                                                                  \
            const float d = h2f(db);                                                                       \
            if (32 * J < n)                                                                                \
                for (int e = 0; e < 32; ++e)                                                               \
                    out[32 * J + e] = __fmul_rn((float)(int8_t)((v[e >> 2] >> (8 * (e & 3))) & 0xFFu), d); \
        }
        SB_Q8_DEQ(0) SB_Q8_DEQ(1) SB_Q8_DEQ(2) SB_Q8_DEQ(3)
#undef SB_Q8_DEQ
    }
}

}  // namespace sabah
