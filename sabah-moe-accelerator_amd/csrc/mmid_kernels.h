// Decode-path kernels: MUL_MAT_ID on the GGUF-layout expert bank, the fused
// gate/up/SiLU of a MoE layer, the routed-expert combine, and the dequantiser.
//
// Every kernel is one workgroup of 256 threads (four wave64s) per tile of R
// consecutive rows of one expert matrix.  A tile is contiguous in HBM
// (rows x row_bytes), so it is staged into LDS with 16-byte coalesced loads,
// decoded from LDS in 32-element items, and dotted against the q8 activation
// row that the same workgroup quantised into LDS in its prologue (ggml's CPU
// quantises src1 once per row; doing it per workgroup costs one L2 read of the
// fp32 row and no extra launch or synchronisation).
//
// Arithmetic per output row, as ggml's vec_dot kernels do it:
//   exact int32 block sum of (weight ints x activation ints) with the block's
//   integer sub-scales, then  c_b = (d_w * d_x) * isum_b  (Q4_K also subtracts
//   (dmin_w * d_x) * msum_b), then the row value = sum over blocks in block
//   order, in fp32.
#pragma once
#include "act_quant.h"
#include "decode_items.h"

namespace sabah {

constexpr int kThreads = 256;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// HBM -> LDS staging of a tile of rows
// ---------------------------------------------------------------------------
__device__ inline void copy_to_lds(uint8_t* dst, const uint8_t* __restrict__ src, int n) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const uintptr_t sa = reinterpret_cast<uintptr_t>(src);
    if ((sa & 15) == 0 && (n & 15) == 0) {
        const u32x4* s = reinterpret_cast<const u32x4*>(src);
        u32x4* d = reinterpret_cast<u32x4*>(dst);
        for (int q = tid; q < (n >> 4); q += nt) d[q] = __builtin_nontemporal_load(s + q);
    } else if ((sa & 3) == 0 && (n & 3) == 0) {
        const uint32_t* s = reinterpret_cast<const uint32_t*>(src);
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
        for (int q = tid; q < (n >> 2); q += nt) d[q] = __builtin_nontemporal_load(s + q);
    } else if ((sa & 1) == 0 && (n & 1) == 0) {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(src);
        uint16_t* d = reinterpret_cast<uint16_t*>(dst);
        for (int q = tid; q < (n >> 1); q += nt) d[q] = s[q];
    } else {
        for (int q = tid; q < n; q += nt) dst[q] = src[q];
    }
}

// rows [0, nrows) of a matrix whose rows are row_stride apart, packed in LDS
// at row_bytes apart
__device__ inline void stage_rows(uint8_t* lds, const uint8_t* src, size_t row_stride, int rb, int nrows) {
    if (row_stride == (size_t)rb) {
        copy_to_lds(lds, src, rb * nrows);
    } else {
        for (int r = 0; r < nrows; ++r) copy_to_lds(lds + r * rb, src + (size_t)r * row_stride, rb);
    }
}

__device__ inline void stage_grid(uint32_t* grid_lds) {
    for (int i = threadIdx.x; i < 512; i += blockDim.x) grid_lds[i] = kIq3sGridDev.e[i];
}

// ---------------------------------------------------------------------------
// Tile mat-vec: per (row, block) fp32 contributions into part[r * nsb + b]
// ---------------------------------------------------------------------------
template <int QT>
__device__ inline void tile_matvec(const uint8_t* tile, int rb, int nrows, int k, const uint8_t* act,
                                   const uint32_t* grid, float* part) {
    constexpr int IPB = block_elems(QT) / 32;   // items per block: 8 (256-blocks) or 1 (Q8_0)
    const ActLayout AL(k, act_type(QT));
    const int NI = k / 32, NSB = NI / IPB;
    const int total = nrows * NI;
    const int16_t* bsum = reinterpret_cast<const int16_t*>(act + AL.off_bsum);
    const float* adx = reinterpret_cast<const float*>(act + AL.off_d);
    for (int base = 0; base < total; base += blockDim.x) {
        const int it = base + (int)threadIdx.x;
        const bool valid = it < total;
        int isum = 0, msum = 0, r = 0, p = 0;
        if (valid) {
            r = it / NI;
            p = it - r * NI;
            const Item item = decode_item<QT>(tile, (uint32_t)(r * rb), p, grid);
            const uint4 a0 = reinterpret_cast<const uint4*>(act)[2 * p];
            const uint4 a1 = reinterpret_cast<const uint4*>(act)[2 * p + 1];
            const uint32_t av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            isum = item_dot<QT>(item, av, bsum, p, msum);
        }
        if constexpr (IPB == 8) {
            // the eight items of a block sit in eight aligned consecutive lanes
            isum += __shfl_xor(isum, 1, 64);
            isum += __shfl_xor(isum, 2, 64);
            isum += __shfl_xor(isum, 4, 64);
            if constexpr (QT == QT_Q4_K) {
                msum += __shfl_xor(msum, 1, 64);
                msum += __shfl_xor(msum, 2, 64);
                msum += __shfl_xor(msum, 4, 64);
            }
        }
        if (valid && (p % IPB) == 0) {
            const int b = p / IPB;
            const float dx = adx[b];
            const float dw = block_d<QT>(tile, (uint32_t)(r * rb), p);
            float c = __fmul_rn(__fmul_rn(dw, dx), (float)isum);
            if constexpr (QT == QT_Q4_K) {
                const float dm = block_dmin<QT>(tile, (uint32_t)(r * rb), p);
                c = __fsub_rn(c, __fmul_rn(__fmul_rn(dm, dx), (float)msum));
            }
            part[r * NSB + b] = c;
        }
    }
}

// fp32 row value = sum of its block contributions in block order
__device__ inline float row_sum(const float* part, int r, int nsb) {
    float s = 0.0f;
    for (int b = 0; b < nsb; ++b) s = __fadd_rn(s, part[r * nsb + b]);
    return s;
}

// ---------------------------------------------------------------------------
// Dynamic LDS plan of one workgroup (computed identically on host and device)
// ---------------------------------------------------------------------------
struct LdsPlan {
    int off_grid, off_act, off_act2, off_tile, off_tile2, off_part, off_part2, bytes;
};

__host__ __device__ inline int align16i(int v) { return (v + 15) & ~15; }

// one or two matrices (gate+up) of type qt/qt2 with k columns and R-row tiles
__host__ __device__ inline LdsPlan make_plan(int qt, int qt2, int k, int R) {
    LdsPlan p{};
    int o = 0;
    p.off_grid = o;
    if (qt == QT_IQ3_S || qt2 == QT_IQ3_S) o += 2048;
    p.off_act = o;
    o += align16i((int)ActLayout(k, act_type(qt)).bytes);
    p.off_act2 = p.off_act;
    if (qt2 > 0 && act_type(qt2) != act_type(qt)) {
        p.off_act2 = o;
        o += align16i((int)ActLayout(k, act_type(qt2)).bytes);
    }
    const int nsb = k / block_elems(qt);
    p.off_tile = o;
    o += align16i((int)row_bytes(qt, k) * R + 16);
    p.off_part = o;
    o += align16i(4 * R * nsb);
    p.off_tile2 = p.off_tile;
    p.off_part2 = p.off_part;
    if (qt2 > 0) {
        p.off_tile2 = o;
        o += align16i((int)row_bytes(qt2, k) * R + 16);
        p.off_part2 = o;
        o += align16i(4 * R * (k / block_elems(qt2)));
    }
    p.bytes = o;
    return p;
}

// ---------------------------------------------------------------------------
// Where a slot's expert matrix lives: a bank base + id * expert_stride, with
// the id read on the device (no host round trip), or a pointer table.
// ---------------------------------------------------------------------------
struct ExpertSrc {
    const uint8_t* base;          // bank base (used when ptrs == nullptr)
    const void* const* ptrs;      // optional [n_tokens][n_slots] pointer table
    size_t expert_stride;
};

struct Routing {
    const uint8_t* ids;           // int32 ids, strided as ggml's ids tensor
    size_t id_stride, token_stride;
    int n_experts;
};

__device__ inline int read_id(const Routing& R, int t, int s) {
    return *reinterpret_cast<const int32_t*>(R.ids + (size_t)t * R.token_stride + (size_t)s * R.id_stride);
}

// resolves the expert matrix of (token t, slot s); returns nullptr for an id
// outside [0, n_experts)
// (a Routing without ids addresses expert 0: a dense matrix such as the shared expert)
__device__ inline const uint8_t* expert_ptr(const ExpertSrc& E, const Routing& R, int t, int s, int n_slots) {
    if (E.ptrs) return reinterpret_cast<const uint8_t*>(E.ptrs[(size_t)t * n_slots + s]);
    const int e = R.ids ? read_id(R, t, s) : 0;
    if (e < 0 || e >= R.n_experts) return nullptr;
    return E.base + (size_t)e * E.expert_stride;
}

// ---------------------------------------------------------------------------
// MUL_MAT_ID (sabah_rt_mul_mat_id_v2 semantics, sabah_rt.cu:2791-2839):
//   dst[t][i][r] = W[ids[t][i]][r] . q8(x[t][i % x_rows])
// grid = (ceil(rows / R), n_ids, n_tokens)
// ---------------------------------------------------------------------------
struct MmidArgs {
    ExpertSrc W;
    Routing rt;
    size_t row_stride;
    const uint8_t* x;
    size_t x_id_stride, x_token_stride;
    int x_rows;
    int n_ids, n_tokens;
    uint8_t* dst;
    size_t dst_id_stride, dst_token_stride;
    int rows, k, R;
    unsigned int* err;            // sticky error word, host-mapped; every writer stores 1
};

template <int QT>
__global__ __launch_bounds__(kThreads) void k_mmid(MmidArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const LdsPlan P = make_plan(QT, 0, a.k, a.R);
    const int t = blockIdx.z, i = blockIdx.y, row0 = blockIdx.x * a.R;
    const int rb = (int)row_bytes(QT, a.k);
    const int nrows = min(a.R, a.rows - row0);
    float* out = reinterpret_cast<float*>(a.dst + (size_t)t * a.dst_token_stride + (size_t)i * a.dst_id_stride) + row0;
    const uint8_t* w = expert_ptr(a.W, a.rt, t, i, a.n_ids);
    if (w == nullptr) {   // uniform across the workgroup
        if (threadIdx.x == 0) *reinterpret_cast<volatile unsigned int*>(a.err) = 1u;
        for (int r = threadIdx.x; r < nrows; r += blockDim.x) out[r] = __builtin_nanf("");
        return;
    }
    stage_rows(smem + P.off_tile, w + (size_t)row0 * a.row_stride, a.row_stride, rb, nrows);
    if constexpr (QT == QT_IQ3_S) stage_grid(reinterpret_cast<uint32_t*>(smem + P.off_grid));
    const float* xr = reinterpret_cast<const float*>(a.x + (size_t)t * a.x_token_stride +
                                                     (size_t)(i % a.x_rows) * a.x_id_stride);
    wg_quantize_row(xr, a.k, act_type(QT), smem + P.off_act);
    __syncthreads();
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    tile_matvec<QT>(smem + P.off_tile, rb, nrows, a.k, smem + P.off_act,
                    reinterpret_cast<const uint32_t*>(smem + P.off_grid), part);
    __syncthreads();
    const int nsb = a.k / block_elems(QT);
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) out[r] = row_sum(part, r, nsb);
}

// ---------------------------------------------------------------------------
// Fused gate/up + SwiGLU of the routed experts (ggml: two MUL_MAT_ID + GLU,
// qwen4exp.cpp:848-862; executor.py:1-16):
//   h[t][s][j] = silu(Wg[e][j] . q8(x[t])) * (Wu[e][j] . q8(x[t]))
// grid = (ceil(d_ff / R), n_slots, n_tokens).  A slot whose expert pointer is
// null is skipped (used for the shared expert, whose h rows go elsewhere).
// ---------------------------------------------------------------------------
struct GateUpArgs {
    ExpertSrc G, U;
    Routing rt;
    const float* x;               // [n_tokens][d_model]
    float* h;                     // [n_tokens][n_slots][d_ff]
    int n_slots, d_model, d_ff, R;
    unsigned int* err;
};

__device__ inline float silu_f32(float v) {
    return __fdiv_rn(v, __fadd_rn(1.0f, expf(-v)));
}

template <int QTG, int QTU>
__global__ __launch_bounds__(kThreads) void k_gate_up(GateUpArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const LdsPlan P = make_plan(QTG, QTU, a.d_model, a.R);
    const int t = blockIdx.z, s = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.d_ff - row0);
    const int rbg = (int)row_bytes(QTG, a.d_model), rbu = (int)row_bytes(QTU, a.d_model);
    float* h = a.h + ((size_t)t * a.n_slots + s) * a.d_ff + row0;
    const uint8_t* wg = expert_ptr(a.G, a.rt, t, s, a.n_slots);
    const uint8_t* wu = expert_ptr(a.U, a.rt, t, s, a.n_slots);
    if (wg == nullptr || wu == nullptr) {
        if (threadIdx.x == 0) *reinterpret_cast<volatile unsigned int*>(a.err) = 1u;
        for (int r = threadIdx.x; r < nrows; r += blockDim.x) h[r] = __builtin_nanf("");
        return;
    }
    stage_rows(smem + P.off_tile, wg + (size_t)row0 * rbg, rbg, rbg, nrows);
    stage_rows(smem + P.off_tile2, wu + (size_t)row0 * rbu, rbu, rbu, nrows);
    if constexpr (QTG == QT_IQ3_S || QTU == QT_IQ3_S) stage_grid(reinterpret_cast<uint32_t*>(smem + P.off_grid));
    const float* xr = a.x + (size_t)t * a.d_model;
    wg_quantize_row(xr, a.d_model, act_type(QTG), smem + P.off_act);
    if (P.off_act2 != P.off_act) wg_quantize_row(xr, a.d_model, act_type(QTU), smem + P.off_act2);
    __syncthreads();
    const uint32_t* grid = reinterpret_cast<const uint32_t*>(smem + P.off_grid);
    float* pg = reinterpret_cast<float*>(smem + P.off_part);
    float* pu = reinterpret_cast<float*>(smem + P.off_part2);
    tile_matvec<QTG>(smem + P.off_tile, rbg, nrows, a.d_model, smem + P.off_act, grid, pg);
    tile_matvec<QTU>(smem + P.off_tile2, rbu, nrows, a.d_model, smem + P.off_act2, grid, pu);
    __syncthreads();
    const int nsg = a.d_model / block_elems(QTG), nsu = a.d_model / block_elems(QTU);
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        const float g = row_sum(pg, r, nsg), u = row_sum(pu, r, nsu);
        h[r] = __fmul_rn(silu_f32(g), u);
    }
}

// ---------------------------------------------------------------------------
// Routed combine (ggml_mul by the router weights, then ggml_add over the slots
// in slot order), plus an optional shared-expert row and residual:
//   out[t][i] = (((y0*w0 + y1*w1) + ...) + y_{n-1}*w_{n-1}) [+ shared[t][i]] [+ resid[t][i]]
// ---------------------------------------------------------------------------
__global__ void k_combine(const float* __restrict__ y, const float* __restrict__ w, const float* __restrict__ shared,
                          const float* resid, float* out, int n_slots, int d_model, int n_tokens, int accumulate) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= d_model || t >= n_tokens) return;
    const float* yt = y + (size_t)t * n_slots * d_model;
    const float* wt = w + (size_t)t * n_slots;
    float acc = __fmul_rn(yt[i], wt[0]);
    for (int s = 1; s < n_slots; ++s) acc = __fadd_rn(acc, __fmul_rn(yt[(size_t)s * d_model + i], wt[s]));
    if (shared) acc = __fadd_rn(acc, shared[(size_t)t * d_model + i]);
    float* o = out + (size_t)t * d_model + i;
    if (resid) acc = __fadd_rn(resid[(size_t)t * d_model + i], acc);
    if (accumulate) acc = __fadd_rn(*o, acc);
    *o = acc;
}

// ---------------------------------------------------------------------------
// Dequantiser through the same item decoders (ggml dequantize_row_* float order)
// grid = ceil(n_rows / R)
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                      int n_rows, int k, int R) {
    extern __shared__ __align__(16) uint8_t smem[];
    const LdsPlan P = make_plan(QT, 0, k, R);
    const int row0 = blockIdx.x * R;
    const int nrows = min(R, n_rows - row0);
    const int rb = (int)row_bytes(QT, k);
    stage_rows(smem + P.off_tile, src + (size_t)row0 * rb, rb, rb, nrows);
    if constexpr (QT == QT_IQ3_S) stage_grid(reinterpret_cast<uint32_t*>(smem + P.off_grid));
    __syncthreads();
    const uint32_t* grid = reinterpret_cast<const uint32_t*>(smem + P.off_grid);
    const uint8_t* tile = smem + P.off_tile;
    const int NI = k / 32;
    for (int it = threadIdx.x; it < nrows * NI; it += blockDim.x) {
        const int r = it / NI, p = it - r * NI;
        const Item item = decode_item<QT>(tile, (uint32_t)(r * rb), p, grid);
        const float d = block_d<QT>(tile, (uint32_t)(r * rb), p);
        const float dm = block_dmin<QT>(tile, (uint32_t)(r * rb), p);
        float* o = dst + (size_t)(row0 + r) * k + 32 * p;
        for (int l = 0; l < 32; ++l) o[l] = item_value<QT>(item, l, d, dm);
    }
}

// ---------------------------------------------------------------------------
// Activation quantiser exposed for byte-level checks: rows of k floats into
// ggml's own block layout (block_q8_0: fp16 d + 32 int8; block_q8_K: f32 d +
// 256 int8 + 16 int16 bsums).  grid = n_rows, one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_quantize_act_ggml(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                                int k, int at) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int r = blockIdx.x;
    wg_quantize_row(x + (size_t)r * k, k, at, smem);
    __syncthreads();
    const ActLayout L(k, at);
    const int qb = block_elems(at), bb = block_bytes(at), nb = k / qb;
    uint8_t* yr = y + (size_t)r * nb * bb;
    const float* d = reinterpret_cast<const float*>(smem + L.off_d);
    for (int q = threadIdx.x; q < k; q += blockDim.x) {
        const int b = q / qb, j = q - b * qb;
        yr[(size_t)b * bb + (at == QT_Q8_K ? 4 : 2) + j] = smem[q];
    }
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        if (at == QT_Q8_K) {
            const float dv = d[b];
            memcpy(yr + (size_t)b * bb, &dv, 4);
            const int16_t* bs = reinterpret_cast<const int16_t*>(smem + L.off_bsum) + 16 * b;
            memcpy(yr + (size_t)b * bb + 260, bs, 32);
        } else {
            const unsigned short hb = __half_as_ushort(__float2half_rn(d[b]));
            yr[(size_t)b * bb] = (uint8_t)(hb & 0xff);
            yr[(size_t)b * bb + 1] = (uint8_t)(hb >> 8);
        }
    }
}

}  // namespace sabah
