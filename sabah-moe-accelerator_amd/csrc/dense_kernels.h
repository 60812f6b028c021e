// A dense (always-on) expert over a batch of tokens: the shared expert of a
// layer at n_tokens > 1 (qwen4exp.cpp:866-887: gate/up + SwiGLU, down,
// scaled by sigmoid(ffn_gate_inp_shexp . x) and added after the routed
// experts).  The token-major kernels run grid z = tokens, so every token's
// workgroups stage the same rows again; here a workgroup stages its rows
// once and dots them with all of its tokens' activations, so each weight row
// is read once per launch (per TB tokens).
//
// Activations arrive quantised (k_quant_rows: x, then h, into ActLayout rows
// act_stride bytes apart), since every workgroup needs all of its tokens'
// rows and quantising them per workgroup would cost more than the dots.
// Each thread is one (token, matrix, row): it walks the row's units in order
// and adds their block contributions to one fp32 sum in block order, the
// order the token-major kernels' row_sum adds the same terms, so the results
// are bit-identical to theirs.
#pragma once
#include "mmid_kernels.h"

namespace sabah {

// contributions of unit us of a row, added to s in block order
template <int QT>
__device__ inline float unit_accumulate(const LdsWindow<QT>& Wn, const uint8_t* tabs, const uint8_t* act, int k,
                                        int us, float s) {
    const ActLayout AL(k, act_type(QT));
    const float* dxa = reinterpret_cast<const float*>(act + AL.off_d);
    const int16_t* bsa = reinterpret_cast<const int16_t*>(act + AL.off_bsum);
    if constexpr (QT == QT_Q8_0 || QT == QT_IQ4_NL || QT == QT_Q5_1) {
        const int16_t* bs = QT == QT_Q5_1 ? reinterpret_cast<const int16_t*>(reinterpret_cast<const float*>(bsa) + 4 * us)
                                          : bsa;
        const uint8_t* chunk = act + (us >> 1) * kActChunkStride + (us & 1) * 128;
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, chunk, dxa + 4 * us, bs);
        const int nb = min(4, k / 32 - 4 * us);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < nb) s = __fadd_rn(s, r.c[j]);
    } else if constexpr (QT == QT_Q2_0) {
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, act + us * kActChunkStride, dxa + 8 * us, bsa);
        const int nc = 2 * min(4, k / 64 - 4 * us);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < nc) s = __fadd_rn(s, r.c[j]);
    } else if constexpr (QT == QT_IQ4_XS) {
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, act + us * kActChunkStride, dxa + us, bsa + 16 * us);
#pragma unroll
        for (int j = 0; j < 8; ++j) s = __fadd_rn(s, r.c[j]);
    } else {
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, act + us * kActChunkStride, dxa + us, bsa + 16 * us);
        s = __fadd_rn(s, r.c[0]);
    }
    return s;
}

struct DenseArgs {
    const uint8_t* w0;            // gate (two-matrix form) or the one matrix: [rows][row bytes], packed
    const uint8_t* w1;            // up (two-matrix form), or nullptr
    const uint8_t* xq;            // [n_tokens] quantised activation rows, act_stride bytes apart
    int act_stride;
    int n_tokens, k, rows;
    int R, TB;                    // rows and tokens per workgroup
    float* out;                   // [n_tokens][rows]: h = silu(g) * u, or y
    const float* sg_w;            // two-matrix form: the shared gate row (or nullptr); its logit
    const float* sg_x;            //   sg_w . sg_x[t] (sg_x [n_tokens][sg_n]) goes to sg_logit[t]
    int sg_n;
    float* sg_logit;              // [n_tokens]; the one-matrix form scales y by sigmoid(sg_logit[t]) (or nullptr)
};

// LDS of a launch beyond the static arrays: the TB activation rows, then the
// per-(token, matrix, row) sums
__host__ __device__ inline int dense_dyn_lds(int TB, int act_stride, int n_mat, int R) {
    return TB * act_stride + align16i(4 * TB * n_mat * R);
}
// 16-byte loads per thread that bring in the activation rows
constexpr int kDenseActLoads = 24;

// grid = (ceil(rows / R), ceil(n_tokens / TB)); TB * NMAT * R <= kThreads and
// the NMAT tiles of R rows stage in one pass (both checked by the host)
template <int QT, int NMAT>
__global__ __launch_bounds__(kThreads) void k_dense_tokens(DenseArgs a) {
    SABAH_STATIC_LDS(QT)
    extern __shared__ __align__(16) uint8_t smem[];
    const int row0 = blockIdx.x * a.R, t0 = blockIdx.y * a.TB;
    const int nrows = min(a.R, a.rows - row0), ntok = min(a.TB, a.n_tokens - t0);
    const int tid = (int)threadIdx.x;
    const size_t rb = row_bytes(QT, a.k);
    uint8_t* act = smem;
    float* res = reinterpret_cast<float*>(smem + a.TB * a.act_stride);
    const TableRegs<QT, kThreads> gr = load_tables<QT, kThreads>(tid);
    const uint8_t* w0 = a.w0 + (size_t)row0 * rb;
    const uint8_t* w1 = NMAT == 2 ? a.w1 + (size_t)row0 * rb : w0;
    auto tile_ptr = [&](int m) { return m ? w1 : w0; };
    TileRun<QT> S{TileWalk<QT>(NMAT, nrows, rb, a.k)};
    tiles_begin(S, tile_ptr);
    // the tokens' activation rows (contiguous), every load issued before the stores
    {
        const int n16 = (ntok * a.act_stride) >> 4;
        const u32x4* src = reinterpret_cast<const u32x4*>(a.xq + (size_t)t0 * a.act_stride);
        u32x4* dst = reinterpret_cast<u32x4*>(act);
        u32x4 v[kDenseActLoads];
#pragma unroll
        for (int i = 0; i < kDenseActLoads; ++i) {
            const int idx = tid + kThreads * i;
            if (idx < n16) v[i] = src[idx];
        }
#pragma unroll
        for (int i = 0; i < kDenseActLoads; ++i) {
            const int idx = tid + kThreads * i;
            if (idx < n16) dst[idx] = v[i];
        }
    }
    store_tables<QT, kThreads>(tabs, gr, tid);
    // the shared gate's logits: workgroup (b, 0) takes tokens b, b + grid.x, ...
    // in the token-major down kernel's order (gate_dot_part, gate_dot_total)
    if (NMAT == 2 && a.sg_w && blockIdx.y == 0) {
        __shared__ float sg_sums[4];
        for (int t = blockIdx.x; t < a.n_tokens; t += gridDim.x) {
            gate_dot_part(a.sg_w, a.sg_x + (size_t)t * a.sg_n, a.sg_n, sg_sums);
            __syncthreads();
            if (tid == 0) a.sg_logit[t] = gate_dot_total(sg_sums);
            __syncthreads();
        }
    }
    pass_store(S, stage, leads);
    __syncthreads();                                        // weights, activations and table in LDS
    // thread = token tt + TB * (matrix m + NMAT * row r)
    const int NUS = units_per_row(QT, a.k);
    if (tid < a.TB * NMAT * a.R) {
        const int q = div_small(tid, __builtin_amdgcn_rcpf((float)a.TB));
        const int tt = tid - q * a.TB;
        const int r = NMAT == 2 ? q >> 1 : q, m = NMAT == 2 ? q & 1 : 0;
        if (tt < ntok && r < nrows) {
            const uint8_t* rowp = stage + 16 * S.cpt * m + leads[m] + (int)((size_t)r * rb) - S.b0;
            const uint8_t* arow = act + tt * a.act_stride;
            float s = 0.0f;
            for (int us = 0; us < NUS; ++us) {
                LdsWindow<QT> Wn;
                Wn.load(rowp + us * UnitFmt<QT>::BYTES);
                s = unit_accumulate<QT>(Wn, tabs, arow, a.k, us, s);
            }
            res[q * a.TB + tt] = s;
        }
    }
    __syncthreads();
    const float rcp_rows = __builtin_amdgcn_rcpf((float)nrows);
    for (int j = tid; j < ntok * nrows; j += kThreads) {
        const int tt = div_small(j, rcp_rows), r = j - tt * nrows;
        float y;
        if constexpr (NMAT == 2) {
            y = __fmul_rn(silu_f32(res[(2 * r) * a.TB + tt]), res[(2 * r + 1) * a.TB + tt]);
        } else {
            y = res[r * a.TB + tt];
            if (a.sg_logit) y = __fmul_rn(y, sigmoid_f32(a.sg_logit[t0 + tt]));
        }
        a.out[(size_t)(t0 + tt) * a.rows + row0 + r] = y;
    }
}

}  // namespace sabah
