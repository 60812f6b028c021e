// Group-major MoE layer for a batch of tokens (prefill).
//
// The token-major kernels read every routed expert matrix once per (token,
// slot) that selects it, as the reference's kernel does (grid z = n_tokens,
// sabah_rt.cu:2791-2839).  Here the (token, slot) pairs are grouped by expert
// on the device, and each expert's rows are read once per layer and applied
// to all of its pairs with int8 MFMA (v_mfma_i32_16x16x32_i8: 16 rows x 16
// pairs x one 32-element sub-block per instruction).  The semantics are
// upstream ggml's sorted MUL_MAT_ID fallback (ggml-cuda.cu:1985-2082): group
// by expert, per-expert matrix product, scatter back, weighted combine.
//
// The integer block sums are exact, and every fp32 step (block scale times
// block sum, the serial sum over blocks, SwiGLU, the slot-ordered combine)
// is the token-major path's, so the results are bit-identical to it.
//
// Kernels of one layer, in stream order:
//   k_group_pairs     ids -> per-expert offsets and the pairs in group order
//   k_quant_rows      x -> q8_K rows (ActLayout), one per pair in group order
//   k_grouped_gate_up h[pos] = silu(Wg[e] . q8(x[t])) * (Wu[e] . q8(x[t]))
//   k_quant_rows      h -> q8_K rows, one per grouped pair
//   k_grouped_down    y[pos] = Wd[e] . q8(h[pos])
//   k_combine         out[t] = [resid +] ((y0 w0 + y1 w1) + ...) [+ shared]
// Supported: gate and up of one type, down of any, each IQ3_S, Q4_K or Q6_K;
// d_model / 256 even and <= 8; d_ff / 256 <= 4.
//
// The same kernels, instantiated with MMID = true, run a grouped MUL_MAT_ID
// (sabah_rt_mul_mat_id_v2 over many tokens): k_group_pairs, k_quant_rows on
// x, then k_grouped_down<QT, true> (k <= 1024, 64-row tiles) or
// k_grouped_gate_up<QT, true> (k <= 2048, two 16-row groups of one matrix in the
// places of gate and up, no SwiGLU), each reading x through the pair's token
// (or its own row when x has one row per slot) and writing dst[t][slot].
#pragma once
#include "mmid_kernels.h"

namespace sabah {

constexpr int kGroupThreads = 1024;
constexpr int kPairTile = 16;                 // pairs per MFMA column tile
constexpr int kGuRows = 16;                   // gate/up rows per workgroup (one MFMA row tile)
constexpr int kDownRows = 64;                 // down rows per workgroup (four MFMA row tiles)
constexpr int kDownBlocks = 4;                // 256-blocks of k per down wave (one wave per row tile)

typedef int v4i32 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Grouping.  Pair p = t * k + s.  off[e] .. off[e+1] are expert e's positions;
// pair_of[pos] is the pair at a position and pos_of[p] the position of a
// pair (-1 for an id outside [0, n_experts), which also sets the error word).
// The order of pairs inside a group is not fixed (LDS atomics): it changes no
// value, only where a pair's rows are kept.
// ---------------------------------------------------------------------------
struct GroupArgs {
    const int32_t* ids;           // [n_tokens][k]
    int n_tokens, k, n_experts;
    int* off;                     // [n_experts + 1]
    int* pair_of;                 // [n_tokens * k]
    int* pos_of;                  // [n_tokens * k]
    unsigned int* err;
    float* poison;                // MUL_MAT_ID: a bad pair's dst row becomes NaN (null: none)
    size_t poison_nb1, poison_nb2;  // dst slot and token strides, bytes
    int poison_rows;
};

// exclusive scan of one int per thread over the workgroup (a multiple of 64
// threads, at most 1024): a shuffle scan per wave, then the wave totals;
// tmp holds 16 ints
__device__ inline int block_exclusive_scan(int v, int* tmp, int& total) {
    const int lane = (int)(threadIdx.x & 63u), wave = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < nw; ++w) {
        const int t = tmp[w];
        before += w < wave ? t : 0;
        total += t;
    }
    __syncthreads();
    return before + x - v;
}

// ids a thread keeps in registers between the histogram and the scatter
// (n_tokens * k up to 8 x 1024); larger batches re-read them
constexpr int kGroupIdRegs = 8;

// one workgroup of kGroupThreads; dynamic LDS: 2 * n_experts + kGroupThreads ints
__global__ __launch_bounds__(kGroupThreads) void k_group_pairs(GroupArgs a) {
    extern __shared__ int glds[];
    const int E = a.n_experts, P = a.n_tokens * a.k, NT = (int)blockDim.x, tid = (int)threadIdx.x;
    int* cnt = glds;
    int* fill = glds + E;
    int* tmp = glds + 2 * E;
    // every id load is issued before any is used (one memory latency, not one per pair)
    const bool in_regs = P <= kGroupIdRegs * NT;
    int idv[kGroupIdRegs];
#pragma unroll
    for (int i = 0; i < kGroupIdRegs; ++i) {
        const int p = tid + NT * i;
        idv[i] = in_regs && p < P ? a.ids[p] : -1;
    }
    for (int e = tid; e < E; e += NT) cnt[e] = 0;
    __syncthreads();
    // f(p, e) for each of the thread's pairs
    auto each_pair = [&](auto&& f) {
        if (in_regs) {
#pragma unroll
            for (int i = 0; i < kGroupIdRegs; ++i)
                if (tid + NT * i < P) f(tid + NT * i, idv[i]);
        } else {
            for (int p = tid; p < P; p += NT) f(p, a.ids[p]);
        }
    };
    each_pair([&](int, int e) {
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    });
    __syncthreads();
    // each thread scans a contiguous run of seg experts
    const int seg = (E + NT - 1) / NT;
    const int e0 = min(E, tid * seg), e1 = min(E, e0 + seg);
    int s = 0;
    for (int e = e0; e < e1; ++e) s += cnt[e];
    int total;
    int run = block_exclusive_scan(s, tmp, total);
    for (int e = e0; e < e1; ++e) {
        fill[e] = run;
        a.off[e] = run;
        run += cnt[e];
    }
    if (tid == 0) a.off[E] = total;
    __syncthreads();
    bool bad = false;
    each_pair([&](int p, int e) {
        if (e >= 0 && e < E) {
            const int pos = atomicAdd(&fill[e], 1);
            a.pair_of[pos] = p;
            a.pos_of[p] = pos;
        } else {
            a.pos_of[p] = -1;
            bad = true;
            if (a.poison) {                                 // error path only: one thread per bad pair
                float* d = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.poison) +
                                                    (size_t)(p / a.k) * a.poison_nb2 + (size_t)(p % a.k) * a.poison_nb1);
                for (int r = 0; r < a.poison_rows; ++r) d[r] = __builtin_nanf("");
            }
        }
    });
    if (bad) *reinterpret_cast<volatile unsigned int*>(a.err) = 1u;
}

// ---------------------------------------------------------------------------
// q8 rows in the kernels' activation layout (ActLayout), n_rows rows of k
// floats.  Each workgroup quantises 16 chunk-rows (one per 16-lane row).
// With `gather`, output row r is input row gather[r] / gdiv, for the rows
// below *count (the grouped pairs: the rows come out in group order).  With
// mfma_order (q8_K only), each chunk's bytes are in the grouped kernels'
// operand order (row16_quant_q8K).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_quant_rows(const float* __restrict__ x, int n_rows, int k, int at,
                                                         uint8_t* __restrict__ out, int out_stride,
                                                         const int* __restrict__ gather, int gdiv,
                                                         const int* __restrict__ count, int mfma_order) {
    const int nch = k / 256;
    const int q = blockIdx.x * (kThreads / 16) + (int)(threadIdx.x >> 4);
    if (q >= n_rows * nch) return;                       // whole 16-lane rows leave together
    const int r = q / nch, c = q - r * nch;
    if (count && r >= *count) return;
    const int src = gather ? gather[r] / gdiv : r;
    const ActBatch B{x, (size_t)k, n_rows, k, at, out, out_stride};
    Act16 v;
    load16(x + (size_t)src * k, c * 256 + 16 * (int)(threadIdx.x & 15u), k, act_vec(B), v);
    quant_chunk(B, v, q, mfma_order != 0);
}

// ---------------------------------------------------------------------------
// MFMA operands.  For v_mfma_i32_16x16x32_i8, lane l holds row (A) or column
// (B) l % 16 and the eight k-values 8 (l / 16) .. +7 of the 32; the int32
// result's lane l holds column l % 16 and rows 4 (l / 16) .. +3.
// ---------------------------------------------------------------------------

// The weights are the B operand (columns = the tile's 16 rows, lane l holding
// row l % 16's eight k-values 8 (l / 16) .. +7 of a sub-block), the pairs'
// activations the A operand; so the int32 result's lane l holds row l % 16
// for pairs 4 (l / 16) .. +3, and the row's sub-block scales and d are the
// lane's own.
//
// What lane quarter q of a staged IQ3_S unit needs for each of the unit's
// eight sub-blocks s: the qs bytes 8s + 2q, 8s + 2q + 1 (grid groups 2q and
// 2q + 1), their ninth index bits (bits 2q, 2q + 1 of qh[s]) and sign
// nibbles (byte 4s + q of the signs); and the unit's sub-block scales and d.
// Read once per block (the unit starts at an even byte).  A group's table
// index is the 16-bit value [qs, h] with h = sign nibble | ninth bit << 4
// (the codebook table's layout), so the fields are packed as the bytes one
// v_perm turns into both indices of a sub-block.
struct Iq3sQuarter {
    uint32_t qs[4];               // halfword s & 1 of qs[s >> 1]: [qs_2q, qs_2q+1] of sub-block s
    uint32_t lh[4];               // halfword s & 1 of lh[s >> 1]: [h_2q, h_2q+1] of sub-block s
    uint32_t sc;                  // the four scale bytes (nibble s: sub-block s)
    uint32_t d;                   // fp16 d (low half)
};
__device__ inline void iq3s_quarter_fields(const uint8_t* unit, int q, Iq3sQuarter& F) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(unit);
#pragma unroll
    for (int p = 0; p < 4; ++p)
        F.qs[p] = (uint32_t)h[1 + 8 * p + q] | (uint32_t)h[5 + 8 * p + q] << 16;   // bytes 2 + 8s + 2q, s = 2p, 2p + 1
    const uint32_t qh[2] = {(uint32_t)h[33] | (uint32_t)h[34] << 16, (uint32_t)h[35] | (uint32_t)h[36] << 16};
    const uint8_t* sg = unit + 74 + q;
    const uint32_t sw[2] = {(uint32_t)sg[0] | (uint32_t)sg[4] << 8 | (uint32_t)sg[8] << 16 | (uint32_t)sg[12] << 24,
                            (uint32_t)sg[16] | (uint32_t)sg[20] << 8 | (uint32_t)sg[24] << 16 | (uint32_t)sg[28] << 24};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        // byte j (sub-block 4k + j): h of group 2q in lo, of group 2q + 1 in hi
        const uint32_t b0 = ((qh[k] >> (2 * q)) << 4) & 0x10101010u;
        const uint32_t b1 = ((qh[k] >> (2 * q + 1)) << 4) & 0x10101010u;
        const uint32_t lo = (sw[k] & 0x0F0F0F0Fu) | b0;
        const uint32_t hi = ((sw[k] >> 4) & 0x0F0F0F0Fu) | b1;
        F.lh[2 * k] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);       // [lo.b0, hi.b0, lo.b1, hi.b1]
        F.lh[2 * k + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);   // [lo.b2, hi.b2, lo.b3, hi.b3]
    }
    F.sc = (uint32_t)h[53] | (uint32_t)h[54] << 16;
    F.d = h[0];
}
// the lane's eight weights of sub-block s (B operand) from the signed codebook table
__device__ inline long iq3s_quarter_operand(const Iq3sQuarter& F, const uint8_t* tabs, int s, int q) {
    (void)q;
    const uint32_t p = 2u * (uint32_t)(s & 1);
    // [qs_2q, h_2q, qs_2q+1, h_2q+1]: the two 16-bit table indices
    const uint32_t sel = (4u + p) | (p << 8) | ((5u + p) << 16) | ((p + 1u) << 24);
    const uint32_t W = __builtin_amdgcn_perm(F.qs[s >> 1], F.lh[s >> 1], sel);
    const uint32_t g0 = lds_u32(tabs, kLdsGrid + lo16_x4(W));
    const uint32_t g1 = lds_u32(tabs, kLdsGrid + (W >> 14));      // h < 32: bits 14, 15 of W are 0
    return (long)(((uint64_t)g1 << 32) | g0);
}

// A dword of a staged unit at any even address (two 16-bit LDS reads)
__device__ inline uint32_t lds_u32_even(const uint8_t* p) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)h[0] | (uint32_t)h[1] << 16;
}

// Q4_K: lane quarter q's eight elements of item j (elements 32j .. 32j + 31)
// are nibbles (low for even j, high for odd) of qs bytes 32 (j / 2) + 8q ..
// +7; the item's 6-bit scale and min (get_scale_min_k4) and the unit's d,
// dmin are the row's.  Unit: d, dmin (4 B), scales (12 B), qs (128 B).
struct Q4kQuarter {
    uint32_t qs[8];               // qs bytes 32p + 8q .. +7 for p = 0..3, two dwords each
    uint32_t sc[3];               // the 12 packed scale/min bytes
    uint32_t dd;                  // fp16 d | fp16 dmin << 16
};
__device__ inline void q4k_quarter_fields(const uint8_t* unit, int q, Q4kQuarter& F) {
    F.dd = lds_u32_even(unit);
#pragma unroll
    for (int i = 0; i < 3; ++i) F.sc[i] = lds_u32_even(unit + 4 + 4 * i);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        F.qs[2 * p] = lds_u32_even(unit + 16 + 32 * p + 8 * q);
        F.qs[2 * p + 1] = lds_u32_even(unit + 20 + 32 * p + 8 * q);
    }
}
__device__ inline long q4k_quarter_operand(const Q4kQuarter& F, int j) {
    const uint64_t w = (uint64_t)F.qs[2 * (j >> 1)] | (uint64_t)F.qs[2 * (j >> 1) + 1] << 32;
    return (long)((w >> (4 * (j & 1))) & 0x0F0F0F0F0F0F0F0Full);
}
// get_scale_min_k4 (ggml) on the 12 scale bytes
__device__ inline void q4k_quarter_scale_min(const Q4kQuarter& F, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = (int)(byte_of(F.sc, j) & 63u);
        mn = (int)(byte_of(F.sc, j + 4) & 63u);
    } else {
        sc = (int)((byte_of(F.sc, j + 4) & 0xFu) | ((byte_of(F.sc, j - 4) >> 6) << 4));
        mn = (int)((byte_of(F.sc, j + 4) >> 4) | ((byte_of(F.sc, j) >> 6) << 4));
    }
}

// Q6_K: item j = half h = j / 4, quarter t = j % 4: the low 4 bits of lane
// quarter q's eight elements are nibbles t / 2 of ql bytes 64h + 32 (t & 1)
// + 8q .. +7, the high 2 bits bits 2t of qh bytes 32h + 8q .. +7; value q6 -
// 32.  The int8 scales (one per 16 elements) and d are the row's.  Unit: ql
// (128 B), qh (64 B), scales (16 B), d (2 B).  The bits are read one half
// at a time (fewer live registers).
struct Q6kQuarter {
    uint32_t sc[4];               // the 16 int8 scales
    uint32_t d;                   // fp16 d (low half)
};
__device__ inline void q6k_quarter_fields(const uint8_t* unit, Q6kQuarter& F) {
#pragma unroll
    for (int i = 0; i < 4; ++i) F.sc[i] = lds_u32_even(unit + 192 + 4 * i);
    F.d = reinterpret_cast<const uint16_t*>(unit + 208)[0];
}
// half h's bits for lane quarter q: ql bytes 64h + 32u + 8q .. +7 (u = 0, 1), qh bytes 32h + 8q .. +7
struct Q6kHalf {
    uint64_t ql[2], qh;
};
__device__ inline void q6k_half_fields(const uint8_t* unit, int h, int q, Q6kHalf& H) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
        H.ql[u] = (uint64_t)lds_u32_even(unit + 64 * h + 32 * u + 8 * q) |
                  (uint64_t)lds_u32_even(unit + 64 * h + 32 * u + 8 * q + 4) << 32;
    H.qh = (uint64_t)lds_u32_even(unit + 128 + 32 * h + 8 * q) | (uint64_t)lds_u32_even(unit + 132 + 32 * h + 8 * q) << 32;
}
// item 4h + t
__device__ inline long q6k_half_operand(const Q6kHalf& H, int t) {
    const uint64_t lo = H.ql[t & 1] >> (4 * (t >> 1)), hi = H.qh >> (2 * t);
    return (long)((lo & 0x0F0F0F0F0F0F0F0Full) | ((hi & 0x0303030303030303ull) << 4));
}
__device__ inline int q6k_quarter_scale(const Q6kQuarter& F, int s16) {
    return (int)(int8_t)((F.sc[s16 >> 2] >> (8 * (s16 & 3))) & 0xFFu);
}

// One pair's activation words for blocks [b0, b1) of a row (this lane's MFMA
// row and k-quarter q), the blocks' scales and, for the K formats, the q8_K
// block sums the lane feeds the side products: Q4_K the two 32-element sums
// of items q and q + 4, Q6_K the 16-element sums q, q + 4, q + 8, q + 12.
// Loaded ahead of the MFMAs that use them, so their latency is paid once.
template <int NBMAX>
struct XRegs {
    long X[NBMAX][8];
    float dx[NBMAX];
    float bsv[NBMAX][4];
};
// The rows are in MFMA operand order (k_quant_rows with mfma_order): the
// lane's eight bytes of sub-blocks 2 t and 2 t + 1 are one 16-byte load.
template <int QT, int NBMAX>
__device__ inline void load_x(XRegs<NBMAX>& R, const uint8_t* xrow, const ActLayout& XL, int b0, int b1, int q) {
    const float* dxrow = reinterpret_cast<const float*>(xrow + XL.off_d);
    const int16_t* bsrow = reinterpret_cast<const int16_t*>(xrow + XL.off_bsum);
#pragma unroll
    for (int j = 0; j < NBMAX; ++j) {
        const int b = min(b0 + j, b1 - 1);                 // blocks past b1 re-read the last one (unused)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 v = *reinterpret_cast<const uint4*>(xrow + b * kActChunkStride + 64 * t + 16 * q);
            R.X[j][2 * t] = (long)((uint64_t)v.y << 32 | v.x);
            R.X[j][2 * t + 1] = (long)((uint64_t)v.w << 32 | v.z);
        }
        R.dx[j] = dxrow[b];
        if constexpr (QT == QT_Q4_K) {
            R.bsv[j][0] = (float)((int)bsrow[16 * b + 2 * q] + (int)bsrow[16 * b + 2 * q + 1]);
            R.bsv[j][1] = (float)((int)bsrow[16 * b + 2 * q + 8] + (int)bsrow[16 * b + 2 * q + 9]);
        } else if constexpr (QT == QT_Q6_K) {
#pragma unroll
            for (int t = 0; t < 4; ++t) R.bsv[j][t] = (float)bsrow[16 * b + q + 4 * t];
        }
    }
}

typedef float v4f32 __attribute__((ext_vector_type(4)));

// 16 rows x 16 pairs over blocks [b0, b1) of a row: per block the row's exact
// integer block sum(s) against the pair, as the token-major unit dot forms
// them, then the same fp32 steps:
//   IQ3_S: bsum = sum_sub ls * (W_sub . x_sub);            c = (d_w d_x) bsum
//   Q4_K:  isum = sum_j sc_j (q_j . x_j), msum = sum_j mn_j bs_j;
//          c = (d_w d_x) isum - (dmin_w d_x) msum
//   Q6_K:  isum = sum_h sc_h (q_h . x_h) - 32 sum_h sc_h bs_h;   c = (d_w d_x) isum
// The weight terms run on int8 MFMA (Q6_K: one per 16-element half, the other
// half's activations zero); the bsum side terms on fp32 MFMA, exact because
// every product and partial sum is an integer below 2^24.  rowp is the
// lane's staged weight row; lanes of a pair past the tile (valid false)
// multiply zeros.  c[blk][i] is for the lane's row and pair 4q + i.  PIN
// (IQ3_S): form the block sum's first half before the second half's MFMAs
// issue, so at most four MFMA results are live (a kernel at 128 VGPRs keeps
// four waves per SIMD without spilling; with more registers to spare, the
// unpinned order overlaps more MFMAs and is faster).
template <int QT, int NBMAX, bool PIN = false, bool MASK = true>
__device__ inline void mfma_blocks(const uint8_t* rowp, const uint8_t* tabs, int b0, int b1, const XRegs<NBMAX>& R,
                                   bool valid_in, int q, float (&c)[NBMAX][4]) {
    constexpr int UB = UnitFmt<QT>::BYTES;
    const bool valid = valid_in || !MASK;
#pragma unroll
    for (int j = 0; j < NBMAX; ++j) {
        const int b = b0 + j;
        if (b >= b1) break;
        const uint8_t* unit = rowp + UB * b;
        const v4i32 z = {0, 0, 0, 0};
        // d_x of the output pairs 4q .. 4q + 3: lanes 4q + i hold them (lane l loads pair l % 16)
        const float dxv = valid ? R.dx[j] : 0.0f;
        auto dx_of = [&](int i) { return __shfl(dxv, 4 * q + i); };
        if constexpr (QT == QT_IQ3_S) {
            Iq3sQuarter F;
            iq3s_quarter_fields(unit, q, F);
            int bs[4] = {0, 0, 0, 0};
#pragma unroll
            for (int sub = 0; sub < 8; ++sub) {
                const long B = iq3s_quarter_operand(F, tabs, sub, q);
                const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(valid ? R.X[j][sub] : 0, B, z, 0, 0, 0);
                const int ls = 2 * (int)((F.sc >> (4 * sub)) & 15u) + 1;
#pragma unroll
                for (int i = 0; i < 4; ++i) bs[i] += __mul24(ls, d[i]);
                if (PIN && sub == 3)
#pragma unroll
                    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(bs[i]));
            }
            const float dw = h2f(F.d);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[j][i] = __fmul_rn(__fmul_rn(dw, dx_of(i)), (float)bs[i]);
        } else if constexpr (QT == QT_Q4_K) {
            Q4kQuarter F;
            q4k_quarter_fields(unit, q, F);
            int isum[4] = {0, 0, 0, 0};
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(valid ? R.X[j][it] : 0, q4k_quarter_operand(F, it),
                                                                       z, 0, 0, 0);
                int sc, mn;
                q4k_quarter_scale_min(F, it, sc, mn);
#pragma unroll
                for (int i = 0; i < 4; ++i) isum[i] += __mul24(sc, d[i]);
            }
            // msum: pairs' item sums (k = the lane's item q, q + 4) x the row's mins
            int sc0, mn0, sc1, mn1;
            q4k_quarter_scale_min(F, q, sc0, mn0);
            q4k_quarter_scale_min(F, q + 4, sc1, mn1);
            v4f32 ms = {0.0f, 0.0f, 0.0f, 0.0f};
            ms = __builtin_amdgcn_mfma_f32_16x16x4f32(valid ? R.bsv[j][0] : 0.0f, (float)mn0, ms, 0, 0, 0);
            ms = __builtin_amdgcn_mfma_f32_16x16x4f32(valid ? R.bsv[j][1] : 0.0f, (float)mn1, ms, 0, 0, 0);
            const float dw = h2f(F.dd), dmin = h2f(F.dd >> 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dxi = dx_of(i);
                c[j][i] = __fsub_rn(__fmul_rn(__fmul_rn(dw, dxi), (float)isum[i]), __fmul_rn(__fmul_rn(dmin, dxi), ms[i]));
            }
        } else {
            static_assert(QT == QT_Q6_K, "grouped formats: IQ3_S, Q4_K, Q6_K");
            Q6kQuarter F;
            q6k_quarter_fields(unit, F);
            const long lo_half = q < 2 ? -1L : 0L;         // the lane's k-values are in the item's first half
            int isum[4] = {0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                Q6kHalf H;
                q6k_half_fields(unit, h, q, H);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int it = 4 * h + t;
                    const long B = q6k_half_operand(H, t);
                    const long X = valid ? R.X[j][it] : 0;
                    const v4i32 da = __builtin_amdgcn_mfma_i32_16x16x32_i8(X & lo_half, B, z, 0, 0, 0);
                    const v4i32 db = __builtin_amdgcn_mfma_i32_16x16x32_i8(X & ~lo_half, B, z, 0, 0, 0);
                    const int sa = q6k_quarter_scale(F, 2 * it), sb = q6k_quarter_scale(F, 2 * it + 1);
#pragma unroll
                    for (int i = 0; i < 4; ++i) isum[i] += __mul24(sa, da[i]) + __mul24(sb, db[i]);
                }
                // the half's sums are formed here, so only its MFMA results are live at a time
                // (otherwise the sums are reassociated past the block's 16 MFMAs, whose
                // results then spill)
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(isum[i]));
            }
            // sum_h sc_h bs_h: pairs' 16-element sums (h = q + 4t) x the row's scales
            v4f32 tb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                tb = __builtin_amdgcn_mfma_f32_16x16x4f32(valid ? R.bsv[j][t] : 0.0f, (float)q6k_quarter_scale(F, q + 4 * t),
                                                         tb, 0, 0, 0);
            const float dw = h2f(F.d);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[j][i] = __fmul_rn(__fmul_rn(dw, dx_of(i)), (float)(isum[i] - 32 * (int)tb[i]));
        }
    }
}

// One IQ3_S block of the lane's row decoded once into MFMA B operands (its
// eight sub-blocks), for a wave that runs the same rows against several pair
// tiles: each tile then costs only its MFMAs and the block sum.
struct Iq3sBlockOps {
    long B[8];
    uint32_t ls[2];               // byte k of ls[p]: sub-block 2k + p's scale 2 sc + 1
    uint32_t d;
};
__device__ inline void iq3s_block_ops(const uint8_t* unit, const uint8_t* tabs, int q, Iq3sBlockOps& O) {
    Iq3sQuarter F;
    iq3s_quarter_fields(unit, q, F);
#pragma unroll
    for (int sub = 0; sub < 8; ++sub) O.B[sub] = iq3s_quarter_operand(F, tabs, sub, q);
    O.ls[0] = ((F.sc & 0x0F0F0F0Fu) << 1) | 0x01010101u;
    O.ls[1] = (((F.sc >> 4) & 0x0F0F0F0Fu) << 1) | 0x01010101u;
    O.d = F.d;
}
// mfma_blocks' IQ3_S block (one block, the same integer sums and fp32 steps)
// from operands decoded by iq3s_block_ops.  Unmasked: lanes of a pair past
// the tile hold the tile's last pair's activations (the row is clamped), so
// their products are finite and reach only that pair's outputs, which the
// epilogue skips.  (Masking there measured no faster; in k_grouped_down the
// masked form is kept: unmasked it measured 205 against 170 us per 512-token
// IQ3_S down, with the same instruction count less the selects.)
__device__ inline void mfma_block_iq3s_ops(const Iq3sBlockOps& O, const XRegs<1>& R, int q, float (&c)[4]) {
    const v4i32 z = {0, 0, 0, 0};
    const float dxv = R.dx[0];
    int bs[4] = {0, 0, 0, 0};
#pragma unroll
    for (int sub = 0; sub < 8; ++sub) {
        const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(R.X[0][sub], O.B[sub], z, 0, 0, 0);
        const int ls = (int)((O.ls[sub & 1] >> (8 * (sub >> 1))) & 0xFFu);
#pragma unroll
        for (int i = 0; i < 4; ++i) bs[i] += __mul24(ls, d[i]);
        if (sub == 3)
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(bs[i]));
    }
    const float dw = h2f(O.d);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __fmul_rn(__fmul_rn(dw, __shfl(dxv, 4 * q + i)), (float)bs[i]);
}

// The same for the wave's block of both matrices (gate and up) against one
// pair tile: the two matrices' MFMAs for a sub-block issue back to back on the
// shared activation operand, so each result has the other MFMA to cover its
// latency before its multiply-adds; the pairs' d_x are shuffled once for both.
// Each matrix's integer sums and fp32 steps are mfma_block_iq3s_ops'.
__device__ inline void mfma_block_iq3s_ops2(const Iq3sBlockOps& O0, const Iq3sBlockOps& O1, const XRegs<1>& R, int q,
                                            float (&c0)[4], float (&c1)[4]) {
    const v4i32 z = {0, 0, 0, 0};
    const float dxv = R.dx[0];
    int bs0[4] = {0, 0, 0, 0}, bs1[4] = {0, 0, 0, 0};
#pragma unroll
    for (int sub = 0; sub < 8; ++sub) {
        const v4i32 d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(R.X[0][sub], O0.B[sub], z, 0, 0, 0);
        const v4i32 d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(R.X[0][sub], O1.B[sub], z, 0, 0, 0);
        const int ls0 = (int)((O0.ls[sub & 1] >> (8 * (sub >> 1))) & 0xFFu);
        const int ls1 = (int)((O1.ls[sub & 1] >> (8 * (sub >> 1))) & 0xFFu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bs0[i] += __mul24(ls0, d0[i]);
            bs1[i] += __mul24(ls1, d1[i]);
        }
        if (sub == 3)
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(bs0[i]), "+v"(bs1[i]));
    }
    const float dw0 = h2f(O0.d), dw1 = h2f(O1.d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float dxi = __shfl(dxv, 4 * q + i);
        c0[i] = __fmul_rn(__fmul_rn(dw0, dxi), (float)bs0[i]);
        c1[i] = __fmul_rn(__fmul_rn(dw1, dxi), (float)bs1[i]);
    }
}

// Staging of a grouped workgroup's weights: n_reg regions (matrices) of
// `bytes` contiguous bytes each, loaded as aligned 16-byte chunks and stored
// in LDS at reg * cap + chunk offset; the region's first byte lands at
// lead[reg] (its address mod 16).  Region m is loaded by threads
// m NT / n_reg .. (m + 1) NT / n_reg - 1, whole waves, so a wave's region and
// its base, lead and chunk count are scalars (one region per thread needs no
// per-lane choice of region).  Each thread makes NL loads, enough when
// NL * NT >= n_reg * cap / 16 (every region's chunks fit in cap); loads past
// a region's last chunk repeat it.  A repeat stores the same bytes to the same
// place, so every store is unconditional (a store under a condition lets the
// compiler sink its load past the table set-up, a whole memory latency late).
// With row_bytes (a multiple of 16) and a region that starts 16-aligned, each
// row lands kRowPad bytes after the last (stage_row_stride): rows 16 B-aligned
// would put rows r and r + 8 of an MFMA operand on the same LDS banks (2-way
// conflicts on the unit field reads for 880-byte IQ3_S rows, 16-way for
// 1152-byte Q4_K rows).  Padded chunks are stored as two 8-byte halves.
constexpr int kRowPad = 8;
__device__ inline int stage_row_stride(int rb, int lead) { return rb + ((rb & 15) == 0 && lead == 0 ? kRowPad : 0); }
template <int NL>
struct GroupStage {
    u32x4 d[NL];
    int off[NL];                  // LDS offset of each load
};
template <int NT, int NL, int NREG>
__device__ inline void group_stage_issue(GroupStage<NL>& G, const uint8_t* const (&src)[NREG], int bytes, int cap,
                                         int* leads, int row_bytes = 0) {
    static_assert(NT % (64 * NREG) == 0, "a region's threads are whole waves");
    constexpr int TR = NT / NREG;                           // threads per region
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    const int m = __builtin_amdgcn_readfirstlane((int)threadIdx.x / TR);
    const uint8_t* s = src[0];
#pragma unroll
    for (int mm = 1; mm < NREG; ++mm)
        if (m == mm) s = src[mm];
    const int t = (int)threadIdx.x - m * TR;
    const int lead = (int)(reinterpret_cast<uintptr_t>(s) & 15);
    const uint8_t* const base = s - lead;
    const int nch = (lead + bytes + 15) >> 4;
    const int rch = row_bytes && stage_row_stride(row_bytes, lead) != row_bytes ? row_bytes >> 4 : 0;   // chunks per padded row
    const float rrcp = __builtin_amdgcn_rcpf((float)max(rch, 1));
    if (t == 0) leads[m] = lead;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int cc = min(t + TR * i, nch - 1);
        G.d[i] = *(g_u32x4*)(base + 16 * cc);
        G.off[i] = m * cap + 16 * cc + (rch ? kRowPad * div_small(cc, rrcp) : 0);
    }
}
template <int NL, bool PADDED = false>
__device__ inline void group_stage_store(const GroupStage<NL>& G, uint8_t* stage) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        if constexpr (PADDED) {                             // 8-byte aligned
            *reinterpret_cast<uint2*>(stage + G.off[i]) = make_uint2(G.d[i].x, G.d[i].y);
            *reinterpret_cast<uint2*>(stage + G.off[i] + 8) = make_uint2(G.d[i].z, G.d[i].w);
        } else {
            *reinterpret_cast<u32x4*>(stage + G.off[i]) = G.d[i];
        }
    }
}
// staging bytes of one region of rows rows x rb bytes, room for its lead
__host__ __device__ constexpr int group_cap(int rows, int rb) { return (rows * rb + 31) & ~15; }

// ---------------------------------------------------------------------------
// Grouped gate/up + SwiGLU.  grid = (d_ff / 16, n_experts), 512 threads.
// Above four 256-blocks of k, wave w takes block w of both matrices, so a
// pair tile's activations for a block are loaded by one wave, once (the
// loads of 16 rows x 8 bytes each are what a workgroup's start waits on);
// up to four blocks, wave w takes block w & 3 of matrix w >> 2.  Each wave
// runs its rows against every 16-pair tile of the expert: IQ3_S rows are
// decoded into MFMA operands once, before the first tile, and kept in
// registers for the rest (an expert with 95 pairs has six tiles); the other
// formats decode the staged rows per tile.  The block results meet in LDS
// and are summed in block order before SwiGLU.  The activation rows are the pairs' rows in group order (k_quant_rows
// with the grouping as its gather), so a pair tile's activations load from
// the group offset alone, at the start.
// ---------------------------------------------------------------------------
constexpr int kGuThreads = 512;
constexpr int kGuMaxBlocks = 8;               // 256-blocks of k: one per wave
// one workgroup's gate and up rows at k <= 2048, and the 16-byte loads per thread that stage them
template <int QT>
struct GuStage {
    // padded rows (measured: IQ3_S gate/up 332 against 346 us, Q4_K 132 against
    // 172 us per 512-token call; Q6_K 235 against 231 us, so not padded)
    static constexpr bool PAD = QT != QT_Q6_K;
    static constexpr int CAP = group_cap(kGuRows, kGuMaxBlocks * UnitFmt<QT>::BYTES + (PAD ? kRowPad : 0));
    static constexpr int LOADS = (2 * (CAP / 16) + kGuThreads - 1) / kGuThreads;
};

struct GroupedGateUpArgs {
    const uint8_t *gate, *up;     // bank bases [n_experts][d_ff][row bytes]
    size_t expert_stride;
    const int* off;
    const int* pair_of;
    int k;                        // slots per token (MMID: n_ids)
    const uint8_t* xq;            // q8_K rows of the pairs in group order, xq_stride bytes apart
    int xq_stride;
    float* h;                     // [pairs in group order][d_ff]
    int d_model, d_ff;
    // MMID: rows 32 b .. 32 b + 31 of the one matrix at gate; out = dst[t][s]
    float* dst;
    size_t dst_nb1, dst_nb2;
};

// dst row of pair p (t = p / n_ids, slot p % n_ids) for the grouped MUL_MAT_ID
__device__ inline float* pair_dst(float* dst, size_t nb1, size_t nb2, int n_ids, int p) {
    return reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(dst) + (size_t)(p / n_ids) * nb2 +
                                    (size_t)(p % n_ids) * nb1);
}

// Column of pair p in row r of a block's partial sums: the row's four 4-pair
// groups in the order g ^ ((r >> 1) & 3), so a wave's 16-byte stores (one row,
// four pairs per lane) and the epilogue's reads (sixteen pairs of two rows
// per half-wave) each fall on distinct LDS banks.
__device__ inline int part_col(int r, int p) { return 4 * ((p >> 2) ^ ((r >> 1) & 3)) + (p & 3); }

template <int QT, bool MMID = false>
__global__ __launch_bounds__(kGuThreads, 4) void k_grouped_gate_up(GroupedGateUpArgs a) {
    constexpr int NT = kGuThreads;
    const int e = blockIdx.y;
    const int g0 = a.off[e], n_e = a.off[e + 1] - g0;
    if (n_e == 0) return;                                  // uniform: the whole workgroup leaves
    __shared__ __align__(16) uint8_t tabs[QT == QT_IQ3_S ? kLdsTables : 16];
    __shared__ int leads[2];
    __shared__ __align__(16) uint8_t stage_mem[16 + 2 * GuStage<QT>::CAP + 16];   // guards: reads past a unit's ends
    __shared__ __align__(16) float part[2][kGuMaxBlocks][kGuRows][kPairTile];
    uint8_t* const stage = stage_mem + 16;
    const int row0 = blockIdx.x * (MMID ? 2 * kGuRows : kGuRows);
    const int nb = a.d_model / 256;
    const size_t rb = row_bytes(QT, a.d_model);
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    const bool both = nb > 4;                              // the wave's block of both matrices
    const int m = both ? 0 : wave >> 2, b = both ? wave : wave & 3;
    const int r = lane & 15, q = lane >> 4, j = lane & 15;
    const int xb = min(b, nb - 1);                         // the block this wave's X covers (a valid one)
    const ActLayout XL(a.d_model, QT_Q8_K);
    const uint8_t* wg = a.gate + (size_t)e * a.expert_stride + (size_t)row0 * rb;
    const uint8_t* wu = MMID ? wg + (size_t)kGuRows * rb : a.up + (size_t)e * a.expert_stride + (size_t)row0 * rb;
    GridRegs<NT> gr;
    if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<NT>((int)threadIdx.x);
    GroupStage<GuStage<QT>::LOADS> G;
    const uint8_t* const src[2] = {wg, wu};
    group_stage_issue<NT, GuStage<QT>::LOADS, 2>(G, src, kGuRows * (int)rb, GuStage<QT>::CAP, leads,
                                                  GuStage<QT>::PAD ? (int)rb : 0);
    auto pair_x = [&](int pt, XRegs<1>& R) {
        const int cnt = min(kPairTile, n_e - pt);
        const uint8_t* xrow = a.xq + (size_t)(g0 + pt + min(j, cnt - 1)) * a.xq_stride;
        load_x<QT>(R, xrow, XL, xb, xb + 1, q);
    };
    XRegs<1> XR;
    pair_x(0, XR);                                          // with the weights
    if constexpr (QT == QT_IQ3_S) store_iq3s_tables<NT>(tabs, gr, (int)threadIdx.x);
    group_stage_store<GuStage<QT>::LOADS, GuStage<QT>::PAD>(G, stage);
    __syncthreads();                                        // staged rows, leads and table written
    auto rstride = [&](int lead) { return GuStage<QT>::PAD ? stage_row_stride((int)rb, lead) : (int)rb; };
    const uint8_t* rowp = stage + GuStage<QT>::CAP * m + leads[m] + r * rstride(leads[m]);
    const uint8_t* rowp1 = stage + GuStage<QT>::CAP + leads[1] + r * rstride(leads[1]);
    // IQ3_S: the wave's block of each of its matrices decoded once, for every pair tile
    Iq3sBlockOps O0, O1;
    if constexpr (QT == QT_IQ3_S) {
        if (b < nb) {
            iq3s_block_ops(rowp + UnitFmt<QT>::BYTES * b, tabs, q, O0);
            if (both) iq3s_block_ops(rowp1 + UnitFmt<QT>::BYTES * b, tabs, q, O1);
        }
    }
    for (int pt = 0; pt < n_e; pt += kPairTile) {
        const int cnt = min(kPairTile, n_e - pt);
        const bool valid = j < cnt;
        if (pt) pair_x(pt, XR);
        // MMID: the epilogue thread's dst row (pair jp = t % 16), loaded before the products
        const int pdst = MMID && threadIdx.x < 256 ? a.pair_of[g0 + pt + min((int)(threadIdx.x & 15u), cnt - 1)] : 0;
        if (b < nb) {
            float c[1][4];
            if (QT == QT_IQ3_S && both) {
                float c1[4];
                mfma_block_iq3s_ops2(O0, O1, XR, q, c[0], c1);
                *reinterpret_cast<float4*>(&part[0][b][r][part_col(r, 4 * q)]) = make_float4(c[0][0], c[0][1], c[0][2], c[0][3]);
                *reinterpret_cast<float4*>(&part[1][b][r][part_col(r, 4 * q)]) = make_float4(c1[0], c1[1], c1[2], c1[3]);
            } else {
                if constexpr (QT == QT_IQ3_S) mfma_block_iq3s_ops(O0, XR, q, c[0]);
                else mfma_blocks<QT, 1, true, false>(rowp, tabs, b, b + 1, XR, valid, q, c);
                *reinterpret_cast<float4*>(&part[m][b][r][part_col(r, 4 * q)]) = make_float4(c[0][0], c[0][1], c[0][2], c[0][3]);
                if (both) {
                    if constexpr (QT == QT_IQ3_S) mfma_block_iq3s_ops(O1, XR, q, c[0]);
                    else mfma_blocks<QT, 1, true, false>(rowp1, tabs, b, b + 1, XR, valid, q, c);
                    *reinterpret_cast<float4*>(&part[1][b][r][part_col(r, 4 * q)]) =
                        make_float4(c[0][0], c[0][1], c[0][2], c[0][3]);
                }
            }
        }
        __syncthreads();
        // thread (row rr, pair jp), pairs fastest: both matrices' block sums in block order
        const int t = (int)threadIdx.x, jp = t & 15, rr = (t >> 4) & 15;
        if (t < 256 && jp < cnt) {
            float g = 0.0f, u = 0.0f;
            const int col = part_col(rr, jp);
            for (int b = 0; b < nb; ++b) {
                g = __fadd_rn(g, part[0][b][rr][col]);
                u = __fadd_rn(u, part[1][b][rr][col]);
            }
            if constexpr (MMID) {
                float* d = pair_dst(a.dst, a.dst_nb1, a.dst_nb2, a.k, pdst);
                d[row0 + rr] = g;
                d[row0 + kGuRows + rr] = u;
            } else {
                a.h[(size_t)(g0 + pt + jp) * a.d_ff + row0 + rr] = __fmul_rn(silu_f32(g), u);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Grouped down.  grid = (d_model / 64, n_experts), 256 threads; wave w owns
// rows 16 w .. 16 w + 15 of the workgroup's 64, over the whole of k.
// ---------------------------------------------------------------------------
// ROWS = 128 (k <= 768): each wave takes two 16-row groups against the same
// activation registers, so a pair tile's activations are loaded once per 32
// rows and the table built once per 128.
template <int QT, int ROWS = kDownRows>
struct DownStage {
    static constexpr int NB = ROWS == kDownRows ? kDownBlocks : 3;       // 256-blocks of k held
    static constexpr int RG = ROWS / (4 * 16);                           // 16-row groups per wave
    static constexpr int CAP = group_cap(ROWS, NB * UnitFmt<QT>::BYTES);
    static constexpr int LOADS = (CAP / 16 + kThreads - 1) / kThreads;
};

struct GroupedDownArgs {
    const uint8_t* down;          // bank base [n_experts][d_model][row bytes]
    size_t expert_stride;
    const int* off;
    const uint8_t* hq;            // q8_K rows per grouped pair, hq_stride bytes apart
    int hq_stride;
    float* y;                     // [pairs in group order][d_model]
    int d_model, d_ff;
    // MMID: the q8 rows are the pairs' input rows in group order; out = dst[t][s]
    const int* pair_of;
    int n_ids;
    float* dst;
    size_t dst_nb1, dst_nb2;
};

template <int QT, bool MMID = false, int ROWS = kDownRows>
__global__ __launch_bounds__(kThreads, 2) void k_grouped_down(GroupedDownArgs a) {
    using DS = DownStage<QT, ROWS>;
    const int e = blockIdx.y;
    const int g0 = a.off[e], n_e = a.off[e + 1] - g0;
    if (n_e == 0) return;
    __shared__ __align__(16) uint8_t tabs[QT == QT_IQ3_S ? kLdsTables : 16];
    __shared__ int leads[1];
    __shared__ __align__(16) uint8_t stage_mem[16 + DS::CAP + 16];
    uint8_t* const stage = stage_mem + 16;
    const int row0 = blockIdx.x * ROWS;
    const int nb = a.d_ff / 256;
    const size_t rb = row_bytes(QT, a.d_ff);
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    const int r = lane & 15, q = lane >> 4, rbase = 16 * DS::RG * wave, j = lane & 15;
    const ActLayout HL(a.d_ff, QT_Q8_K);
    GridRegs<kThreads> gr;
    if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<kThreads>((int)threadIdx.x);
    GroupStage<DS::LOADS> G;
    const uint8_t* const src[1] = {a.down + (size_t)e * a.expert_stride + (size_t)row0 * rb};
    group_stage_issue<kThreads, DS::LOADS, 1>(G, src, ROWS * (int)rb, DS::CAP, leads);
    auto pair_x = [&](int pt, XRegs<DS::NB>& R) {
        const int cnt = min(kPairTile, n_e - pt);
        const uint8_t* hrow = a.hq + (size_t)(g0 + pt + min(j, cnt - 1)) * a.hq_stride;
        load_x<QT>(R, hrow, HL, 0, nb, q);
    };
    if constexpr (QT == QT_IQ3_S) store_iq3s_tables<kThreads>(tabs, gr, (int)threadIdx.x);
    group_stage_store(G, stage);
    __syncthreads();                                        // staged rows, lead and table written
    const uint8_t* rowp = stage + leads[0] + (size_t)(rbase + r) * rb;
    XRegs<DS::NB> XR;
    for (int pt = 0; pt < n_e; pt += kPairTile) {
        const int cnt = min(kPairTile, n_e - pt);
        const bool valid = j < cnt;
        pair_x(pt, XR);
        // MMID: the dst rows of the lane's four pairs, loaded now so the stores
        // after the products do not wait for them
        int pidx[4] = {0, 0, 0, 0};
        if constexpr (MMID)
#pragma unroll
            for (int i = 0; i < 4; ++i) pidx[i] = a.pair_of[g0 + pt + min(4 * q + i, cnt - 1)];
#pragma unroll
        for (int rg = 0; rg < DS::RG; ++rg) {
            float c[DS::NB][4];
            mfma_blocks<QT, DS::NB>(rowp + (size_t)(16 * rg) * rb, tabs, 0, nb, XR, valid, q, c);
            // the lane's row for pairs 4q .. 4q + 3
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (4 * q + i >= cnt) break;
                float acc = 0.0f;
#pragma unroll
                for (int jj = 0; jj < DS::NB; ++jj)
                    if (jj < nb) acc = __fadd_rn(acc, c[jj][i]);
                const int pi = g0 + pt + 4 * q + i;
                float* out = MMID ? pair_dst(a.dst, a.dst_nb1, a.dst_nb2, a.n_ids, pidx[i])
                                  : a.y + (size_t)pi * a.d_model;
                out[row0 + rbase + 16 * rg + r] = acc;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Combine in slot order, as k_down_combine does:
//   out[t][i] = [resid[t][i] +] ((y(t,0)[i] w0 + y(t,1)[i] w1) + ...) [+ shared[t][i]]
// grid = (ceil(d_model / (256 VW)), n_tokens); a token with an invalid id gets NaN.
// ---------------------------------------------------------------------------
struct CombineArgs {
    const float* y;               // [pairs in group order][d_model]
    const int* pos_of;            // [n_tokens * k]
    const float* w;               // [n_tokens][k]
    const float* shared;          // optional [n_tokens][d_model]
    const float* resid;           // optional [n_tokens][d_model]
    float* out;                   // [n_tokens][d_model] (may alias resid)
    int k, d_model;
};

// VW elements per thread (4 when d_model % 4 == 0 and out, resid, shared
// are 16-byte aligned, else 1); up to kCombineSlots slots' rows are all
// loaded before the first is added (one memory latency per thread, not one
// per slot); more slots take a loop.
constexpr int kCombineSlots = 16;
template <int VW>
struct CombineVec {
    float v[VW];
};
template <int VW>
__device__ inline CombineVec<VW> combine_load(const float* p) {
    CombineVec<VW> r;
    if constexpr (VW == 4) {
        const float4 x = *reinterpret_cast<const float4*>(p);
        r.v[0] = x.x; r.v[1] = x.y; r.v[2] = x.z; r.v[3] = x.w;
    } else {
        r.v[0] = *p;
    }
    return r;
}
template <int VW>
__global__ __launch_bounds__(kThreads) void k_combine(CombineArgs a) {
    const int t = blockIdx.y, i = VW * (blockIdx.x * kThreads + (int)threadIdx.x);
    if (i >= a.d_model) return;
    const int* pos = a.pos_of + (size_t)t * a.k;
    const float* wt = a.w + (size_t)t * a.k;
    bool bad = false;
    for (int s = 0; s < a.k; ++s) bad |= pos[s] < 0;
    CombineVec<VW> acc;
    if (bad) {
#pragma unroll
        for (int e = 0; e < VW; ++e) acc.v[e] = __builtin_nanf("");
    } else {
        auto yrow = [&](int s) { return combine_load<VW>(a.y + (size_t)pos[s] * a.d_model + i); };
        auto add = [&](int s, const CombineVec<VW>& y) {
            const float w = wt[s];
#pragma unroll
            for (int e = 0; e < VW; ++e) acc.v[e] = s == 0 ? __fmul_rn(y.v[e], w) : __fadd_rn(acc.v[e], __fmul_rn(y.v[e], w));
        };
        if (a.k <= kCombineSlots) {
            CombineVec<VW> y[kCombineSlots];
#pragma unroll
            for (int s = 0; s < kCombineSlots; ++s)
                if (s < a.k) y[s] = yrow(s);
#pragma unroll
            for (int s = 0; s < kCombineSlots; ++s)
                if (s < a.k) add(s, y[s]);
        } else {
            for (int s = 0; s < a.k; ++s) add(s, yrow(s));
        }
        if (a.shared) {
            const CombineVec<VW> sh = combine_load<VW>(a.shared + (size_t)t * a.d_model + i);
#pragma unroll
            for (int e = 0; e < VW; ++e) acc.v[e] = __fadd_rn(acc.v[e], sh.v[e]);
        }
        if (a.resid) {
            const CombineVec<VW> r = combine_load<VW>(a.resid + (size_t)t * a.d_model + i);
#pragma unroll
            for (int e = 0; e < VW; ++e) acc.v[e] = __fadd_rn(r.v[e], acc.v[e]);
        }
    }
    float* o = a.out + (size_t)t * a.d_model + i;
    if constexpr (VW == 4) *reinterpret_cast<float4*>(o) = make_float4(acc.v[0], acc.v[1], acc.v[2], acc.v[3]);
    else *o = acc.v[0];
}

}  // namespace sabah
