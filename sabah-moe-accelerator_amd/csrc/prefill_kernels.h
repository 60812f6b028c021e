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
//   k_quant_rows      x -> q8_K rows (ActLayout), one per token
//   k_grouped_gate_up h[pos] = silu(Wg[e] . q8(x[t])) * (Wu[e] . q8(x[t]))
//   k_quant_rows      h -> q8_K rows, one per grouped pair
//   k_grouped_down    y[pos] = Wd[e] . q8(h[pos])
//   k_combine         out[t] = [resid +] ((y0 w0 + y1 w1) + ...) [+ shared]
// Supported: IQ3_S gate, up and down; d_model / 256 even and <= 8; d_ff / 256 <= 4.
//
// The same kernels, instantiated with MMID = true, run a grouped MUL_MAT_ID
// (sabah_rt_mul_mat_id_v2 over many tokens): k_group_pairs, k_quant_rows on
// x, then k_grouped_down<true> (k <= 1024, 64-row tiles) or
// k_grouped_gate_up<true> (k <= 2048, two 16-row groups of one matrix in the
// places of gate and up, no SwiGLU), each reading x through the pair's token
// (or its own row when x has one row per slot) and writing dst[t][slot].
#pragma once
#include "mmid_kernels.h"

namespace sabah {

constexpr int kGroupThreads = 1024;
constexpr int kPairTile = 16;                 // pairs per MFMA column tile
constexpr int kGuRows = 16;                   // gate/up rows per workgroup (one MFMA row tile)
constexpr int kDownRows = 64;                 // down rows per workgroup (four MFMA row tiles)
constexpr int kGuBlocksPerWave = 4;           // 256-blocks of k per gate/up wave (two waves per matrix)
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

// exclusive scan of one int per thread over the workgroup; tmp holds blockDim.x ints
__device__ inline int block_exclusive_scan(int v, int* tmp, int& total) {
    const int i = (int)threadIdx.x, n = (int)blockDim.x;
    tmp[i] = v;
    __syncthreads();
    for (int o = 1; o < n; o <<= 1) {
        const int x = i >= o ? tmp[i - o] : 0;
        __syncthreads();
        tmp[i] += x;
        __syncthreads();
    }
    total = tmp[n - 1];
    const int r = tmp[i] - v;
    __syncthreads();
    return r;
}

// one workgroup of kGroupThreads; dynamic LDS: 2 * n_experts + kGroupThreads ints
__global__ __launch_bounds__(kGroupThreads) void k_group_pairs(GroupArgs a) {
    extern __shared__ int glds[];
    const int E = a.n_experts, P = a.n_tokens * a.k;
    int* cnt = glds;
    int* fill = glds + E;
    int* tmp = glds + 2 * E;
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = a.ids[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // each thread scans a contiguous run of seg experts
    const int seg = (E + (int)blockDim.x - 1) / (int)blockDim.x;
    const int e0 = min(E, (int)threadIdx.x * seg), e1 = min(E, e0 + seg);
    int s = 0;
    for (int e = e0; e < e1; ++e) s += cnt[e];
    int total;
    int run = block_exclusive_scan(s, tmp, total);
    for (int e = e0; e < e1; ++e) {
        fill[e] = run;
        a.off[e] = run;
        run += cnt[e];
    }
    if (threadIdx.x == 0) a.off[E] = total;
    __syncthreads();
    bool bad = false;
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = a.ids[p];
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
    }
    if (bad) *reinterpret_cast<volatile unsigned int*>(a.err) = 1u;
}

// ---------------------------------------------------------------------------
// q8 rows in the kernels' activation layout (ActLayout), n_rows rows of k
// floats.  Each workgroup quantises 16 chunk-rows (one per 16-lane row).
// With `gather`, output row r is input row gather[r] / gdiv, for the rows
// below *count (the grouped pairs: the rows come out in group order).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_quant_rows(const float* __restrict__ x, int n_rows, int k, int at,
                                                         uint8_t* __restrict__ out, int out_stride,
                                                         const int* __restrict__ gather, int gdiv,
                                                         const int* __restrict__ count) {
    const int nch = k / 256;
    const int q = blockIdx.x * (kThreads / 16) + (int)(threadIdx.x >> 4);
    if (q >= n_rows * nch) return;                       // whole 16-lane rows leave together
    const int r = q / nch, c = q - r * nch;
    if (count && r >= *count) return;
    const int src = gather ? gather[r] / gdiv : r;
    const ActBatch B{x, (size_t)k, n_rows, k, at, out, out_stride};
    Act16 v;
    load16(x + (size_t)src * k, c * 256 + 16 * (int)(threadIdx.x & 15u), k, act_vec(B), v);
    quant_chunk(B, v, q);
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
// Read once per block (the unit starts at an even byte).
struct Iq3sQuarter {
    uint32_t qs[4];               // halfword s of qs[s >> 1]: the lane's two qs bytes of sub-block s
    uint32_t qh[2];               // qh bytes 0..7
    uint32_t sg[2];               // byte s of sg[s >> 2]: the lane's sign byte of sub-block s
    uint32_t sc;                  // the four scale bytes (nibble s: sub-block s)
    uint32_t d;                   // fp16 d (low half)
};
__device__ inline void iq3s_quarter_fields(const uint8_t* unit, int q, Iq3sQuarter& F) {
    const uint16_t* h = reinterpret_cast<const uint16_t*>(unit);
#pragma unroll
    for (int p = 0; p < 4; ++p)
        F.qs[p] = (uint32_t)h[1 + 8 * p + q] | (uint32_t)h[5 + 8 * p + q] << 16;   // bytes 2 + 8s + 2q, s = 2p, 2p + 1
    F.qh[0] = (uint32_t)h[33] | (uint32_t)h[34] << 16;
    F.qh[1] = (uint32_t)h[35] | (uint32_t)h[36] << 16;
    const uint8_t* sg = unit + 74 + q;
    F.sg[0] = (uint32_t)sg[0] | (uint32_t)sg[4] << 8 | (uint32_t)sg[8] << 16 | (uint32_t)sg[12] << 24;
    F.sg[1] = (uint32_t)sg[16] | (uint32_t)sg[20] << 8 | (uint32_t)sg[24] << 16 | (uint32_t)sg[28] << 24;
    F.sc = (uint32_t)h[53] | (uint32_t)h[54] << 16;
    F.d = h[0];
}
// the lane's eight weights of sub-block s (B operand) from the signed codebook table
__device__ inline long iq3s_quarter_operand(const Iq3sQuarter& F, const uint8_t* tabs, int s, int q) {
    const uint32_t qs2 = (F.qs[s >> 1] >> (16 * (s & 1))) & 0xFFFFu;
    const uint32_t qh2 = (F.qh[s >> 2] >> (8 * (s & 3) + 2 * q)) & 3u;
    const uint32_t sgb = (F.sg[s >> 2] >> (8 * (s & 3))) & 0xFFu;
    const uint32_t i0 = (qs2 & 0xFFu) + 256u * ((sgb & 15u) + 16u * (qh2 & 1u));
    const uint32_t i1 = (qs2 >> 8) + 256u * ((sgb >> 4) + 16u * (qh2 >> 1));
    const uint32_t g0 = lds_u32(tabs, kLdsGrid + 4u * i0), g1 = lds_u32(tabs, kLdsGrid + 4u * i1);
    return (long)(((uint64_t)g1 << 32) | g0);
}

// the staged tiles' loads only (no decode): tiles_begin issued them
template <int QT>
__device__ inline void tiles_stage(TileRun<QT>& S, uint8_t* stage, int* leads) {
    pass_store(S, stage, leads);
}

// One pair's activation words for blocks [b0, b1) of a row (this lane's MFMA
// row and k-quarter q), and the blocks' scales.  Loaded ahead of the MFMAs
// that use them, so their latency is paid once.
template <int NBMAX>
struct XRegs {
    long X[NBMAX][8];
    float dx[NBMAX];
};
template <int NBMAX>
__device__ inline void load_x(XRegs<NBMAX>& R, const uint8_t* xrow, const float* dxrow, int b0, int b1, int q) {
#pragma unroll
    for (int j = 0; j < NBMAX; ++j) {
        const int b = min(b0 + j, b1 - 1);                 // blocks past b1 re-read the last one (unused)
#pragma unroll
        for (int sub = 0; sub < 8; ++sub)
            R.X[j][sub] = *reinterpret_cast<const long*>(xrow + b * kActChunkStride + 32 * sub + 8 * q);
        R.dx[j] = dxrow[b];
    }
}

// 16 rows x 16 pairs over blocks [b0, b1) of a row: per block, the exact int32
// block sum sum_sub ls * (W_sub . x_sub), then c = (d_w * d_x) * bsum.  rowp is
// the lane's staged weight row (decoded into the B operand as it is used);
// lanes of a pair past the tile (valid false) multiply zeros.  c[blk][i] is
// for the lane's row and pair 4q + i.
template <int NBMAX>
__device__ inline void mfma_blocks(const uint8_t* rowp, const uint8_t* tabs, int b0, int b1, const XRegs<NBMAX>& R,
                                   bool valid, int q, float (&c)[NBMAX][4]) {
#pragma unroll
    for (int j = 0; j < NBMAX; ++j) {
        const int b = b0 + j;
        if (b >= b1) break;
        Iq3sQuarter F;
        iq3s_quarter_fields(rowp + 110 * b, q, F);
        int bs[4] = {0, 0, 0, 0};
#pragma unroll
        for (int sub = 0; sub < 8; ++sub) {
            v4i32 z = {0, 0, 0, 0};
            const long B = iq3s_quarter_operand(F, tabs, sub, q);
            const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(valid ? R.X[j][sub] : 0, B, z, 0, 0, 0);
            const int ls = 2 * (int)((F.sc >> (4 * sub)) & 15u) + 1;
#pragma unroll
            for (int i = 0; i < 4; ++i) bs[i] += __mul24(ls, d[i]);
        }
        // d_x of the output pairs 4q .. 4q + 3: lanes 4q + i hold them (lane l loads pair l % 16)
        const float dxv = valid ? R.dx[j] : 0.0f;
        const float dw = h2f(F.d);
#pragma unroll
        for (int i = 0; i < 4; ++i) c[j][i] = __fmul_rn(__fmul_rn(dw, __shfl(dxv, 4 * q + i)), (float)bs[i]);
    }
}

// ---------------------------------------------------------------------------
// Grouped gate/up + SwiGLU.  grid = (d_ff / 16, n_experts), 512 threads.
// Wave w: matrix w >> 2 (gate, up), blocks [b0, b1) of k for quarter w & 3.
// Each wave runs its 16 rows x blocks against every 16-pair tile of the
// expert, decoding the staged rows into MFMA operands as it goes; the
// quarters' block results meet in LDS and are summed in block order before
// SwiGLU.  The activation rows are the pairs' rows in group order (k_quant_rows
// with the grouping as its gather), so a pair tile's activations load from
// the group offset alone, at the start.
// ---------------------------------------------------------------------------
constexpr int kGuThreads = 512;
constexpr int kGuWaveBlocks = 2;              // 256-blocks of k per wave (four waves per matrix)
constexpr int kGuMaxBlocks = 4 * kGuWaveBlocks;
// weight staging: both matrices' 16 rows at k <= 2048, each at any lead
constexpr int kGuStageBytes = 2 * 16 * (kGuRows * kGuMaxBlocks * 110 / 16 + 2);

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

template <bool MMID = false>
__global__ __launch_bounds__(kGuThreads, 4) void k_grouped_gate_up(GroupedGateUpArgs a) {
    constexpr int QT = QT_IQ3_S, NT = kGuThreads;
    const int e = blockIdx.y;
    const int g0 = a.off[e], n_e = a.off[e + 1] - g0;
    if (n_e == 0) return;                                  // uniform: the whole workgroup leaves
    __shared__ __align__(16) uint8_t tabs[kLdsTables];
    __shared__ int leads[2];
    __shared__ __align__(16) uint8_t stage_mem[16 + kGuStageBytes + 16];   // guards: the decoder reads past a unit's ends
    __shared__ __align__(16) float part[2][kGuMaxBlocks][kGuRows][kPairTile];
    uint8_t* const stage = stage_mem + 16;
    const int row0 = blockIdx.x * (MMID ? 2 * kGuRows : kGuRows);
    const int nb = a.d_model / 256, bpw = (nb + 3) / 4;
    const size_t rb = row_bytes(QT, a.d_model);
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    const int m = wave >> 2, r = lane & 15, q = lane >> 4, j = lane & 15;
    const int b0 = min(nb, (wave & 3) * bpw), b1 = min(nb, b0 + bpw);
    const int xb0 = min(b0, nb - 1), xb1 = max(b1, xb0 + 1);      // the blocks this wave's X covers (valid ones)
    const ActLayout XL(a.d_model, QT_Q8_K);
    GridRegs<NT> gr = load_grid_regs<NT>((int)threadIdx.x);
    const uint8_t* wg = a.gate + (size_t)e * a.expert_stride + (size_t)row0 * rb;
    const uint8_t* wu = MMID ? wg + (size_t)kGuRows * rb : a.up + (size_t)e * a.expert_stride + (size_t)row0 * rb;
    auto tile_ptr = [&](int mm) { return mm ? wu : wg; };
    TileRun<QT, NT> S{TileWalk<QT, NT>(2, kGuRows, rb, a.d_model)};
    tiles_begin(S, tile_ptr);
    auto pair_x = [&](int pt, XRegs<kGuWaveBlocks>& R) {
        const int cnt = min(kPairTile, n_e - pt);
        const uint8_t* xrow = a.xq + (size_t)(g0 + pt + min(j, cnt - 1)) * a.xq_stride;
        load_x(R, xrow, reinterpret_cast<const float*>(xrow + XL.off_d), xb0, xb1, q);
    };
    XRegs<kGuWaveBlocks> XR;
    pair_x(0, XR);                                          // with the weights
    store_iq3s_tables<NT>(tabs, gr, (int)threadIdx.x);
    pass_store(S, stage, leads);
    __syncthreads();                                        // staged rows and table written
    const uint8_t* rowp = stage + 16 * S.cpt * m + leads[m] + (size_t)r * rb;
    for (int pt = 0; pt < n_e; pt += kPairTile) {
        const int cnt = min(kPairTile, n_e - pt);
        const bool valid = j < cnt;
        if (pt) pair_x(pt, XR);
        float c[kGuWaveBlocks][4];
        mfma_blocks<kGuWaveBlocks>(rowp, tabs, b0, b1, XR, valid, q, c);
#pragma unroll
        for (int jj = 0; jj < kGuWaveBlocks; ++jj)
            if (b0 + jj < b1)
#pragma unroll
                for (int i = 0; i < 4; ++i) part[m][b0 + jj][r][4 * q + i] = c[jj][i];
        __syncthreads();
        // thread (pair jp, row rr), rows fastest: both matrices' block sums in block order
        const int t = (int)threadIdx.x, rr = t & 15, jp = (t >> 4) & 15;
        if (t < 256 && jp < cnt) {
            float g = 0.0f, u = 0.0f;
            for (int b = 0; b < nb; ++b) {
                g = __fadd_rn(g, part[0][b][rr][jp]);
                u = __fadd_rn(u, part[1][b][rr][jp]);
            }
            if constexpr (MMID) {
                float* d = pair_dst(a.dst, a.dst_nb1, a.dst_nb2, a.k, a.pair_of[g0 + pt + jp]);
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

template <bool MMID = false>
__global__ __launch_bounds__(kThreads) void k_grouped_down(GroupedDownArgs a) {
    constexpr int QT = QT_IQ3_S;
    const int e = blockIdx.y;
    const int g0 = a.off[e], n_e = a.off[e + 1] - g0;
    if (n_e == 0) return;
    SABAH_STATIC_LDS(QT)
    const int row0 = blockIdx.x * kDownRows;
    const int nb = a.d_ff / 256;
    const size_t rb = row_bytes(QT, a.d_ff);
    const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63u);
    const int r = lane & 15, q = lane >> 4, rbase = 16 * wave, j = lane & 15;
    const ActLayout HL(a.d_ff, QT_Q8_K);
    GridRegs<kThreads> gr = load_grid_regs<kThreads>((int)threadIdx.x);
    const uint8_t* wd = a.down + (size_t)e * a.expert_stride + (size_t)row0 * rb;
    auto tile_ptr = [&](int) { return wd; };
    TileRun<QT> S{TileWalk<QT>(1, kDownRows, rb, a.d_ff)};
    tiles_begin(S, tile_ptr);
    auto pair_x = [&](int pt, XRegs<kDownBlocks>& R) {
        const int cnt = min(kPairTile, n_e - pt);
        const int pos = g0 + pt + min(j, cnt - 1);
        const uint8_t* hrow = a.hq + (size_t)pos * a.hq_stride;
        load_x(R, hrow, reinterpret_cast<const float*>(hrow + HL.off_d), 0, nb, q);
    };
    store_iq3s_tables<kThreads>(tabs, gr, (int)threadIdx.x);
    tiles_stage(S, stage, leads);
    __syncthreads();                                        // staged rows and table written
    const uint8_t* rowp = stage + leads[0] + (size_t)(rbase + r) * rb;
    XRegs<kDownBlocks> XR;
    for (int pt = 0; pt < n_e; pt += kPairTile) {
        const int cnt = min(kPairTile, n_e - pt);
        const bool valid = j < cnt;
        pair_x(pt, XR);
        float c[kDownBlocks][4];
        mfma_blocks<kDownBlocks>(rowp, tabs, 0, nb, XR, valid, q, c);
        // the lane's row for pairs 4q .. 4q + 3
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (4 * q + i >= cnt) break;
            float acc = 0.0f;
#pragma unroll
            for (int jj = 0; jj < kDownBlocks; ++jj)
                if (jj < nb) acc = __fadd_rn(acc, c[jj][i]);
            const int pi = g0 + pt + 4 * q + i;
            float* out = MMID ? pair_dst(a.dst, a.dst_nb1, a.dst_nb2, a.n_ids, a.pair_of[pi])
                              : a.y + (size_t)pi * a.d_model;
            out[row0 + rbase + r] = acc;
        }
    }
}

// ---------------------------------------------------------------------------
// Combine in slot order, as k_down_combine does:
//   out[t][i] = [resid[t][i] +] ((y(t,0)[i] w0 + y(t,1)[i] w1) + ...) [+ shared[t][i]]
// grid = (ceil(d_model / 256), n_tokens); a token with an invalid id gets NaN.
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

__global__ __launch_bounds__(kThreads) void k_combine(CombineArgs a) {
    const int t = blockIdx.y, i = blockIdx.x * kThreads + (int)threadIdx.x;
    if (i >= a.d_model) return;
    const int* pos = a.pos_of + (size_t)t * a.k;
    const float* wt = a.w + (size_t)t * a.k;
    bool bad = false;
    for (int s = 0; s < a.k; ++s) bad |= pos[s] < 0;
    float* o = a.out + (size_t)t * a.d_model + i;
    if (bad) {
        *o = __builtin_nanf("");
        return;
    }
    float acc = __fmul_rn(a.y[(size_t)pos[0] * a.d_model + i], wt[0]);
    for (int s = 1; s < a.k; ++s) acc = __fadd_rn(acc, __fmul_rn(a.y[(size_t)pos[s] * a.d_model + i], wt[s]));
    if (a.shared) acc = __fadd_rn(acc, a.shared[(size_t)t * a.d_model + i]);
    if (a.resid) acc = __fadd_rn(a.resid[(size_t)t * a.d_model + i], acc);
    *o = acc;
}

}  // namespace sabah
