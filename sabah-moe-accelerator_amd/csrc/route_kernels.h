// Router gating on the device: the softmax -> top-k -> renormalise step that
// ggml's graph runs before MUL_MAT_ID (qwen4exp.cpp:848-862, build_moe_ffn with
// LLAMA_EXPERT_GATING_FUNC_TYPE_SOFTMAX and norm_w; upstream fuses the same
// ops as topk-moe, ggml-cuda.cu:3390-3405).  Per token, in ggml's CPU order:
//   m = max(l);  e_i = exp(l_i - m);  S = sum e_i (double);  p_i = e_i * (float)(1 / S)
//   ids = the n_used largest p, descending (ties: the lower index first)
//   w_j = p[ids_j];  with norm_w: w_j = w_j / (float)(sum_j w_j (double, in j order))
//   with w_scale != 1: w_j = w_j * w_scale
// One workgroup of 256 threads per token; thread v owns experts v, v + 256, ...
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sabah {

constexpr int kRouteThreads = 256;
constexpr int kRouteMaxPerThread = 16;      // n_experts <= 4096
constexpr int kRouteMaxUsed = 64;

struct RouteArgs {
    const float* logits;          // [n_tokens][n_experts]
    int32_t* ids;                 // [n_tokens][n_used]
    float* w;                     // [n_tokens][n_used]
    int n_experts, n_used, norm_w;
    float w_scale;
};

// A candidate as one 64-bit key: the probability's bits (monotonic for
// p >= 0) above the complemented index, so the larger key is the larger p and,
// among equal p, the lower index.  0 marks no candidate (every real key has a
// nonzero low word).
__device__ inline uint64_t route_key(float p, int i) {
    return ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}

template <int CTRL>
__device__ inline uint32_t route_dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ inline void route_max_step(uint32_t& hi, uint32_t& lo) {
    const uint32_t h = route_dpp<CTRL>(hi), l = route_dpp<CTRL>(lo);
    const bool gt = h > hi || (h == hi && l > lo);
    hi = gt ? h : hi;
    lo = gt ? l : lo;
}
// the largest key of the wave, returned to every lane: DPP within each
// 16-lane row, then the four row results through readlane
__device__ inline uint64_t route_wave_max(uint64_t k) {
    uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
    route_max_step<0xB1>(hi, lo);       // quad_perm [1,0,3,2]
    route_max_step<0x4E>(hi, lo);       // quad_perm [2,3,0,1]
    route_max_step<0x141>(hi, lo);      // row_half_mirror
    route_max_step<0x140>(hi, lo);      // row_mirror
    uint64_t best = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint64_t v = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)hi, 16 * r) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)lo, 16 * r);
        best = v > best ? v : best;
    }
    return best;
}

// PER = experts per thread (n_experts <= 256 PER), a compile-time bound so a
// thread's loops cover only its own experts
template <int PER>
__global__ __launch_bounds__(kRouteThreads) void k_route(RouteArgs a) {
    __shared__ float s_max[4];
    __shared__ double s_sum[4];
    __shared__ uint64_t s_best[2][4];
    __shared__ float s_w[kRouteMaxUsed];
    __shared__ int s_id[kRouteMaxUsed];
    const int t = blockIdx.x, v = (int)threadIdx.x, wave = v >> 6, lane = v & 63;
    const float* l = a.logits + (size_t)t * a.n_experts;
    float e[PER];
    int n = 0;
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = v + kRouteThreads * j;
        e[j] = i < a.n_experts ? l[i] : -__builtin_inff();
        if (i < a.n_experts) { m = fmaxf(m, e[j]); n = j + 1; }
    }
    // the maximum (exact in any order)
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) m = fmaxf(m, __shfl_xor(m, k));
    if (lane == 0) s_max[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    // exp and the double sum.  The terms are floats in (0, 1] and there are at
    // most 2^12 of them, so the double sum is exact, and the same in any
    // order, while every term is at least 2^-17; smaller terms round it below
    // float resolution
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        if (j < n && v + kRouteThreads * j < a.n_experts) {
            e[j] = expf(__fsub_rn(e[j], m));
            sum += (double)e[j];
        } else {
            e[j] = -1.0f;                               // below every probability: never selected
        }
    }
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) sum += __shfl_xor(sum, k);
    if (lane == 0) s_sum[wave] = sum;
    __syncthreads();
    const float inv = (float)(1.0 / (((s_sum[0] + s_sum[1]) + s_sum[2]) + s_sum[3]));
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (e[j] >= 0.0f) e[j] = __fmul_rn(e[j], inv);
    // top n_used: one workgroup argmax per pick (one barrier; the wave
    // results alternate between two slots), the winner struck out
    uint64_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) key[j] = e[j] >= 0.0f ? route_key(e[j], v + kRouteThreads * j) : 0;
    for (int k = 0; k < a.n_used; ++k) {
        uint64_t c = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) c = key[j] > c ? key[j] : c;
        c = route_wave_max(c);
        if (lane == 0) s_best[k & 1][wave] = c;
        __syncthreads();
        uint64_t b = s_best[k & 1][0];
#pragma unroll
        for (int q = 1; q < 4; ++q) b = s_best[k & 1][q] > b ? s_best[k & 1][q] : b;
        const int bi = (int)(0xFFFFFFFFu - (uint32_t)b);
        if (v == 0) {
            s_w[k] = __uint_as_float((uint32_t)(b >> 32));
            s_id[k] = bi;
        }
        if ((bi & (kRouteThreads - 1)) == v) {
#pragma unroll
            for (int j = 0; j < PER; ++j)
                if (j == (bi >> 8)) key[j] = 0;
        }
    }
    __syncthreads();                                    // s_w, s_id complete
    if (v == 0) {
        float s = 1.0f;
        if (a.norm_w) {
            double d = 0.0;
            for (int k = 0; k < a.n_used; ++k) d += (double)s_w[k];
            s = (float)d;
        }
        for (int k = 0; k < a.n_used; ++k) {
            float wk = a.norm_w ? __fdiv_rn(s_w[k], s) : s_w[k];
            if (a.w_scale != 1.0f) wk = __fmul_rn(wk, a.w_scale);
            a.w[(size_t)t * a.n_used + k] = wk;
            a.ids[(size_t)t * a.n_used + k] = s_id[k];
        }
    }
}

}  // namespace sabah
