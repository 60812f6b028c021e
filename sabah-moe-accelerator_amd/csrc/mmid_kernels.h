// Decode-path kernels on the GGUF-layout expert bank: MUL_MAT_ID (the v2
// operator), fused gate/up + SwiGLU, fused down + routed combine, the
// dequantiser, and the activation quantiser exposed for byte checks.
//
// Work split: one lane per unit (a 256-element super-block, or four Q8_0
// blocks) of a weight row; a 256-thread workgroup owns a tile of rows.  Each
// lane first issues the loads of its unit (HBM -> VGPRs), then the workgroup
// quantises its activation row(s) into LDS while those loads are in flight,
// then every lane decodes its unit and dots it with the q8 activations.
// Per-row results are formed from per-block contributions summed in block
// order in fp32, as ggml's vec_dot does.
#pragma once
#include "act_quant.h"
#include "unit_decode.h"

namespace sabah {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// expert addressing
// ---------------------------------------------------------------------------
struct ExpertSrc {
    const uint8_t* base;          // bank base (used when ptrs == nullptr)
    const void* const* ptrs;      // optional [n_tokens][n_slots] pointer table
    size_t expert_stride;
};

struct Routing {
    const uint8_t* ids;           // int32 ids, strided as ggml's ids tensor (nullptr: expert 0)
    size_t id_stride, token_stride;
    int n_experts;
};

__device__ inline int read_id(const Routing& R, int t, int s) {
    return *reinterpret_cast<const int32_t*>(R.ids + (size_t)t * R.token_stride + (size_t)s * R.id_stride);
}

// expert matrix of (token t, slot s), or nullptr for an id outside [0, n_experts)
__device__ inline const uint8_t* expert_ptr(const ExpertSrc& E, const Routing& R, int t, int s, int n_slots) {
    if (E.ptrs) return reinterpret_cast<const uint8_t*>(E.ptrs[(size_t)t * n_slots + s]);
    const int e = R.ids ? read_id(R, t, s) : 0;
    if (e < 0 || e >= R.n_experts) return nullptr;
    return E.base + (size_t)e * E.expert_stride;
}

// Per-lane form for a table or id array that is present (E.ptrs or R.ids):
// the routing word of (t, s) is read with two unconditional 4-byte loads
// (the id is read twice), and resolved in a separate step, so a kernel can
// issue other loads before it waits for these.
struct SlotWord {
    uint32_t lo, hi;
};
__device__ inline SlotWord load_slot_word(const ExpertSrc& E, const Routing& R, int t, int s, int n_slots) {
    const bool tbl = E.ptrs != nullptr;
    const uint8_t* p = tbl ? reinterpret_cast<const uint8_t*>(E.ptrs + (size_t)t * n_slots + s)
                           : R.ids + (size_t)t * R.token_stride + (size_t)s * R.id_stride;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    return SlotWord{q[0], q[tbl ? 1 : 0]};
}
__device__ inline const uint8_t* resolve_slot_word(const ExpertSrc& E, const Routing& R, const SlotWord& w) {
    if (E.ptrs) return reinterpret_cast<const uint8_t*>(((uint64_t)w.hi << 32) | w.lo);
    const int e = (int)w.lo;
    if (e < 0 || e >= R.n_experts) return nullptr;
    return E.base + (size_t)e * E.expert_stride;
}

__device__ inline void flag_error(unsigned int* err) {
    if (threadIdx.x == 0) *reinterpret_cast<volatile unsigned int*>(err) = 1u;
}

// ---------------------------------------------------------------------------
// Tile staging.  A workgroup's weights are n_mat "tiles": the same rows
// [row0, row0 + nrows) of n_mat expert matrices (gate and up; the routed
// slots' down matrices; one matrix for MUL_MAT_ID), or single rows when rows
// are not packed.  Every tile holds the same number of units, in row-major
// unit order, at contiguous bytes.  The workgroup walks them in passes of V
// units per tile: a pass copies each tile's byte range HBM -> LDS, then all
// four waves decode the staged units.
//
// The copy uses direct-to-LDS loads (global_load_lds_dwordx4).  The
// compiler makes any later LDS access of a wave wait for that wave's
// outstanding direct-to-LDS loads, so the work is split by wave: waves 0-1
// ("DMA waves") issue the copy, waves 2-3 ("worker waves") meanwhile
// quantise the activations and build the IQ3_S tables.  A tile's bytes are
// copied in 1 KB segments (one load instruction of a wave: 64 lanes x 16
// consecutive bytes); a segment's address is wave-uniform.  Tile t occupies
// segments [t*spt, (t+1)*spt) of the staging area, starting `lead` (its HBM
// address mod 16) bytes into its first segment, so staged bytes keep their
// HBM alignment mod 16; lanes past a tile's last 16-byte chunk re-load that
// chunk into bytes that are never read.
// ---------------------------------------------------------------------------
constexpr int kDmaWaves = 2;
constexpr int kWorkBase = 64 * kDmaWaves;                       // first worker thread
constexpr int kWorkThreads = kThreads - kWorkBase;
constexpr int kSegBytes = 1024;
constexpr int kStageSegs = 32;
constexpr int kStageBytes = kSegBytes * kStageSegs;             // 32 KB per workgroup
constexpr int kStageGuard = 16;
constexpr int kMaxTiles = kStageSegs;                           // at least one segment per tile
static_assert(kDmaWaves == 2, "stage_segments deals segments to two waves");

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// segments per tile of tile_bytes (any lead)
__host__ __device__ inline int tile_segs(int tile_bytes) { return (tile_bytes + 30 + kSegBytes - 1) / kSegBytes; }
// units per tile per pass: the largest V with n_mat * tile_segs(V * unit bytes) <= kStageSegs
__host__ __device__ inline int pass_units(int n_mat, int unit_bytes) {
    return max(1, (kSegBytes * (kStageSegs / n_mat) - 30) / unit_bytes);
}

// DMA wave `wave` issues its share (every kDmaWaves-th segment) of the copy
// of n tiles of pass_bytes each; tile t's pass starts at HBM address
// tile_ptr(t) + b0 (tile_ptr is called with wave-uniform t).
template <typename TilePtr>
__device__ inline void stage_segments(uint8_t* stage, TilePtr tile_ptr, int n, int pass_bytes, int b0, int wave) {
    const int spt = tile_segs(pass_bytes);
    const int lane = (int)(threadIdx.x & 63u);
    for (int t = 0; t < n; ++t) {
        const uint8_t* p = tile_ptr(t) + b0;
        const int lead = (int)(reinterpret_cast<uintptr_t>(p) & 15);
        const int last = (lead + pass_bytes - 1) >> 4;
        const uint8_t* base = p - lead;
        for (int j = (t * spt + wave) & 1; j < spt; j += kDmaWaves) {   // segment t*spt + j is wave (t*spt + j) % 2's
            const int c = min(64 * j + lane, last);
            __builtin_amdgcn_global_load_lds((glb_void_t*)(base + 16 * c),
                                             (lds_void_t*)(stage + kSegBytes * (t * spt + j)), 16, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------
// LDS plan (identical on host and device):
//   [IQ3_S tables][tile leads][guard | staging | guard][activations][partials]
// ---------------------------------------------------------------------------
struct Plan {
    int off_lead, off_stage, off_act, act_bytes, n_act, off_part, bytes;
};

__host__ __device__ inline int align16i(int v) { return (v + 15) & ~15; }

// n_act activation rows of k elements for weight type qt; part = n_part floats
__host__ __device__ inline Plan make_plan(int qt, int k, int n_act, int n_part) {
    Plan p{};
    int o = (qt == QT_IQ3_S) ? kLdsTables : 0;
    p.off_lead = o;
    o += 4 * kMaxTiles;
    p.off_stage = o + kStageGuard;
    o += kStageGuard + kStageBytes + kStageGuard;
    p.off_act = o;
    p.act_bytes = align16i((int)ActLayout(k, act_type(qt)).bytes);
    p.n_act = n_act;
    o += p.act_bytes * n_act;
    p.off_part = o;
    o += align16i(4 * n_part);
    p.bytes = o;
    return p;
}

// Q8_0 rows need only be whole 32-element blocks: their last unit may hold 1..3 blocks
__host__ __device__ inline int units_per_row(int qt, int k) { return qt == QT_Q8_0 ? (k + 127) / 128 : k / 256; }
__host__ __device__ inline int contribs_per_row(int qt, int k) { return k / block_elems(qt); }   // ggml blocks

// Rows per workgroup: about one unit per lane, with the n_mat tiles staged in
// one pass where a row fits.
__host__ __device__ inline int rows_per_wg(int qt, int k, int n_mat) {
    const int nus = units_per_row(qt, k);
    const int by_lanes = kThreads / (n_mat * nus);
    const int by_stage = (kSegBytes * (kStageSegs / n_mat) - 30) / (int)row_bytes(qt, k);
    return max(1, min(by_lanes, by_stage));
}

// bytes of unit us of a row of k elements
template <int QT>
__device__ inline int unit_len(int k, int us) {
    if constexpr (QT == QT_Q8_0) return 34 * min(4, k / 32 - 4 * us);
    return UnitFmt<QT>::BYTES;
}

// dot of one unit (unit index us of its row) with activation row `act`; the
// unit's per-block contributions go to part_row
template <int QT>
__device__ inline void unit_into_part(const UnitWindow<QT>& Wn, const uint8_t* smem, const uint8_t* act, int k, int us,
                                      float* part_row) {
    const ActLayout AL(k, act_type(QT));
    const float* dxa = reinterpret_cast<const float*>(act + AL.off_d);
    const int16_t* bsa = reinterpret_cast<const int16_t*>(act + AL.off_bsum);
    if constexpr (QT == QT_Q8_0) {
        const uint8_t* chunk = act + (us >> 1) * kActChunkStride + (us & 1) * 128;
        const UnitDot<QT> r = unit_dot<QT>(Wn, smem, chunk, dxa + 4 * us, bsa);
        const int nb = min(4, k / 32 - 4 * us);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < nb) part_row[4 * us + j] = r.c[j];
    } else {
        const uint8_t* chunk = act + us * kActChunkStride;
        const UnitDot<QT> r = unit_dot<QT>(Wn, smem, chunk, dxa + us, bsa + 16 * us);
        part_row[us] = r.c[0];
    }
}

__device__ inline float row_sum(const float* part_row, int n) {
    float s = 0.0f;
    for (int b = 0; b < n; ++b) s = __fadd_rn(s, part_row[b]);
    return s;
}

// One workgroup's tiles.  Tile t is matrix tile_ptr(t) from its first row on
// (row0 already folded into the pointer): `nrows` rows of k elements at rb
// bytes, so its unit v = r * NUS + us sits at byte r * rb + us * unit bytes.
// Activations of tile t: act0 + t * act_stride (act_stride 0: one shared
// row).  Contributions of unit (t, r, us) go to part + (t * part_rows + r) * NCB.
template <int QT>
struct TileWalk {
    static constexpr int UB = UnitFmt<QT>::BYTES;
    int n_mat, NUS, NCB, total, V;
    size_t rb;
    __device__ TileWalk(int n_mat_, int nrows, size_t rb_, int k)
        : n_mat(n_mat_), NUS(units_per_row(QT, k)), NCB(contribs_per_row(QT, k)), total(nrows * NUS),
          V(pass_units(n_mat_, UB)), rb(rb_) {}
    __device__ int byte_of(int v) const { return (int)((size_t)(v / NUS) * rb) + (v % NUS) * UB; }
    __device__ int pass_bytes(int v0) const { return byte_of(min(v0 + V, total)) - byte_of(v0); }
};

// DMA waves, before the first pass: record each tile's lead (lane l of wave 0
// holds tile l's pointer in lane_tile) and issue the first pass's copy.
template <int QT, typename TilePtr>
__device__ inline void tiles_begin(const TileWalk<QT>& T, uint8_t* stage, int* leads, const uint8_t* lane_tile,
                                   TilePtr tile_ptr, int wave) {
    if (threadIdx.x < (unsigned)T.n_mat) leads[threadIdx.x] = (int)(reinterpret_cast<uintptr_t>(lane_tile) & 15);
    stage_segments(stage, tile_ptr, T.n_mat, T.pass_bytes(0), 0, wave);
}

// All waves: decode the staged pass, then walk the remaining passes.
template <int QT, typename TilePtr>
__device__ inline void tiles_finish(const TileWalk<QT>& T, const uint8_t* smem, uint8_t* stage, const int* leads,
                                    TilePtr tile_ptr, int wave, int k, const uint8_t* act0, int act_stride,
                                    int part_rows, float* part) {
    for (int v0 = 0;;) {
        const int nv = min(T.V, T.total - v0);
        const int b0 = T.byte_of(v0);
        const int spt = tile_segs(T.pass_bytes(v0));
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int u = threadIdx.x; u < T.n_mat * nv; u += blockDim.x) {
            const int t = u / nv, v = v0 + (u - t * nv);
            const int r = v / T.NUS, us = v - r * T.NUS;
            const int lead = (leads[t] + b0) & 15;
            UnitWindow<QT> Wn;
            Wn.load_lds(stage + kSegBytes * spt * t + lead + (T.byte_of(v) - b0));
            unit_into_part<QT>(Wn, smem, act0 + t * act_stride, k, us, part + (t * part_rows + r) * T.NCB);
        }
        v0 += T.V;
        __syncthreads();   // the pass's units are decoded (and its partials written)
        if (v0 >= T.total) break;
        if (wave < kDmaWaves) stage_segments(stage, tile_ptr, T.n_mat, T.pass_bytes(v0), T.byte_of(v0), wave);
    }
}

__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// wave-uniform copy of lane `src`'s 64-bit pointer
__device__ inline const uint8_t* read_lane_ptr(const uint8_t* p, int src) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src);
    return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// activation rounds prefetched by the worker waves (more are loaded late)
constexpr int kRoundsX = 2;   // one row: up to 16 chunks of 256 (k <= 4096)
constexpr int kRoundsH = 4;   // slot rows: up to 32 chunk-rows (n_slots * ceil(d_ff / 256))

// ---------------------------------------------------------------------------
// MUL_MAT_ID (sabah_rt_mul_mat_id_v2 semantics, sabah_rt.cu:2791-2839):
//   dst[t][i][r] = W[ids[t][i]][r] . q8(x[t][i % x_rows])
// grid = (ceil(rows / R), n_ids, n_tokens).  Rows packed at row_stride form
// one tile; rows row_stride > row bytes apart are one tile each (R <= kMaxTiles).
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
    const int NCB = contribs_per_row(QT, a.k);
    const Plan P = make_plan(QT, a.k, 1, a.R * NCB);
    const int t = blockIdx.z, i = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.rows - row0);
    const size_t rb = row_bytes(QT, a.k);
    const int wave = wave_id();
    float* out = reinterpret_cast<float*>(a.dst + (size_t)t * a.dst_token_stride + (size_t)i * a.dst_id_stride) + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    uint8_t* stage = smem + P.off_stage;
    int* leads = reinterpret_cast<int*>(smem + P.off_lead);
    const float* xr = reinterpret_cast<const float*>(a.x + (size_t)t * a.x_token_stride +
                                                     (size_t)(i % a.x_rows) * a.x_id_stride);
    const ActBatch xb{xr, 0, 1, a.k, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    GridRegs<kWorkThreads> gr;
    if (wave >= kDmaWaves) {   // worker loads first; the expert id is a scalar load with its own counter
        act_prefetch<kRoundsX>(xb, xa, kWorkBase);
        if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<kWorkThreads>((int)threadIdx.x - kWorkBase);
    }
    const uint8_t* w = expert_ptr(a.W, a.rt, t, i, a.n_ids);
    if (w == nullptr) {   // uniform across the workgroup
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += blockDim.x) out[r] = __builtin_nanf("");
        return;
    }
    w += (size_t)row0 * a.row_stride;
    const bool packed = a.row_stride == rb;
    auto tile_ptr = [&](int r) { return packed ? w : w + (size_t)r * a.row_stride; };
    const TileWalk<QT> T(packed ? 1 : nrows, packed ? nrows : 1, rb, a.k);
    if (wave < kDmaWaves) {
        tiles_begin(T, stage, leads, tile_ptr((int)threadIdx.x), tile_ptr, wave);
    } else {
        if constexpr (QT == QT_IQ3_S) store_iq3s_tables<kWorkThreads>(smem, gr, (int)threadIdx.x - kWorkBase);
        act_quantize<kRoundsX>(xb, xa, kWorkBase);
    }
    tiles_finish(T, smem, stage, leads, tile_ptr, wave, a.k, act, 0, packed ? a.R : 1, part);
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) out[r] = row_sum(part + r * NCB, NCB);
}

// ---------------------------------------------------------------------------
// Fused gate/up + SwiGLU of the routed experts (ggml: two MUL_MAT_ID + GLU,
// qwen4exp.cpp:848-862; executor.py:1-16):
//   h[t][s][j] = silu(Wg[e][j] . q8(x[t])) * (Wu[e][j] . q8(x[t]))
// grid = (ceil(d_ff / R), n_slots, n_tokens); tiles = gate rows, up rows
// ---------------------------------------------------------------------------
struct GateUpArgs {
    ExpertSrc G, U;
    Routing rt;
    const float* x;               // [n_tokens][d_model]
    float* h;                     // [n_tokens][n_slots][d_ff]
    int n_slots, d_model, d_ff, R;
    unsigned int* err;
};

__device__ inline float silu_f32(float v) { return __fdiv_rn(v, __fadd_rn(1.0f, expf(-v))); }

template <int QT>
__global__ __launch_bounds__(kThreads) void k_gate_up(GateUpArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int NCB = contribs_per_row(QT, a.d_model);
    const Plan P = make_plan(QT, a.d_model, 1, 2 * a.R * NCB);
    const int t = blockIdx.z, s = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.d_ff - row0);
    const size_t rb = row_bytes(QT, a.d_model);
    const int wave = wave_id();
    float* h = a.h + ((size_t)t * a.n_slots + s) * a.d_ff + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    uint8_t* stage = smem + P.off_stage;
    int* leads = reinterpret_cast<int*>(smem + P.off_lead);
    const ActBatch xb{a.x + (size_t)t * a.d_model, 0, 1, a.d_model, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    GridRegs<kWorkThreads> gr;
    if (wave >= kDmaWaves) {
        act_prefetch<kRoundsX>(xb, xa, kWorkBase);
        if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<kWorkThreads>((int)threadIdx.x - kWorkBase);
    }
    const uint8_t* wg = expert_ptr(a.G, a.rt, t, s, a.n_slots);
    const uint8_t* wu = expert_ptr(a.U, a.rt, t, s, a.n_slots);
    if (wg == nullptr || wu == nullptr) {
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += blockDim.x) h[r] = __builtin_nanf("");
        return;
    }
    wg += (size_t)row0 * rb;
    wu += (size_t)row0 * rb;
    auto tile_ptr = [&](int m) { return m ? wu : wg; };
    const TileWalk<QT> T(2, nrows, rb, a.d_model);
    if (wave < kDmaWaves) {
        tiles_begin(T, stage, leads, threadIdx.x ? wu : wg, tile_ptr, wave);
    } else {
        if constexpr (QT == QT_IQ3_S) store_iq3s_tables<kWorkThreads>(smem, gr, (int)threadIdx.x - kWorkBase);
        act_quantize<kRoundsX>(xb, xa, kWorkBase);
    }
    tiles_finish(T, smem, stage, leads, tile_ptr, wave, a.d_model, act, 0, a.R, part);
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        const float g = row_sum(part + r * NCB, NCB);
        const float up = row_sum(part + (a.R + r) * NCB, NCB);
        h[r] = __fmul_rn(silu_f32(g), up);
    }
}

// ---------------------------------------------------------------------------
// Fused down projection + routed combine (ggml: MUL_MAT_ID on h, ggml_mul by
// the router weights, ggml_add over the slots in slot order), plus optional
// shared-expert rows and residual:
//   out[t][i] = [resid[t][i] +] ((y0*w0 + y1*w1) + ...) [+ shared[t][i]]
//   y_s[i] = Wd[e_s][i] . q8(h[t][s])
// grid = (ceil(d_model / R), n_tokens); tiles = rows of each slot's expert
// (n_slots <= kMaxTiles)
// ---------------------------------------------------------------------------
struct DownArgs {
    ExpertSrc D;
    Routing rt;
    const float* h;               // [n_tokens][n_slots][d_ff]
    const float* w;               // [n_tokens][n_slots] router weights
    const float* shared;          // optional [n_tokens][d_model]
    const float* resid;           // optional [n_tokens][d_model]
    float* out;                   // [n_tokens][d_model] (may alias resid)
    int n_slots, d_model, d_ff, R, accumulate;
    unsigned int* err;
};

template <int QT>
__global__ __launch_bounds__(kThreads) void k_down_combine(DownArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int NCB = contribs_per_row(QT, a.d_ff);
    const Plan P = make_plan(QT, a.d_ff, a.n_slots, a.n_slots * a.R * NCB);
    const int t = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.d_model - row0);
    const size_t rb = row_bytes(QT, a.d_ff);
    const int wave = wave_id();
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    uint8_t* stage = smem + P.off_stage;
    int* leads = reinterpret_cast<int*>(smem + P.off_lead);
    // lane s of every wave holds slot s's tile (lanes past n_slots repeat the
    // last slot); a slot with an invalid id stages expert 0's rows, never
    // used: the output is poisoned.  The id loads go first, so waiting for
    // them does not wait for the activation loads.
    const int lane = (int)(threadIdx.x & 63u);
    const SlotWord sw = load_slot_word(a.D, a.rt, t, min(lane, a.n_slots - 1), a.n_slots);
    const ActBatch hb{a.h + (size_t)t * a.n_slots * a.d_ff, (size_t)a.d_ff, a.n_slots, a.d_ff, act_type(QT), act,
                      P.act_bytes};
    ActRegs<kRoundsH> ha;
    GridRegs<kWorkThreads> gr;
    if (wave >= kDmaWaves) {
        act_prefetch<kRoundsH>(hb, ha, kWorkBase);
        if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<kWorkThreads>((int)threadIdx.x - kWorkBase);
    }
    const uint8_t* e = resolve_slot_word(a.D, a.rt, sw);
    const bool bad = __any(e == nullptr);
    const uint8_t* mine = (e ? e : a.D.base) + (size_t)row0 * rb;
    auto tile_ptr = [&](int m) { return read_lane_ptr(mine, m); };
    const TileWalk<QT> T(a.n_slots, nrows, rb, a.d_ff);
    if (wave < kDmaWaves) {
        tiles_begin(T, stage, leads, mine, tile_ptr, wave);
    } else {
        if constexpr (QT == QT_IQ3_S) store_iq3s_tables<kWorkThreads>(smem, gr, (int)threadIdx.x - kWorkBase);
        act_quantize<kRoundsH>(hb, ha, kWorkBase);
    }
    tiles_finish(T, smem, stage, leads, tile_ptr, wave, a.d_ff, act, P.act_bytes, a.R, part);
    float* o = a.out + (size_t)t * a.d_model + row0;
    if (bad) {
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += blockDim.x) o[r] = __builtin_nanf("");
        return;
    }
    const float* wt = a.w + (size_t)t * a.n_slots;
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        float acc = __fmul_rn(row_sum(part + r * NCB, NCB), wt[0]);
        for (int s = 1; s < a.n_slots; ++s)
            acc = __fadd_rn(acc, __fmul_rn(row_sum(part + (s * a.R + r) * NCB, NCB), wt[s]));
        if (a.shared) acc = __fadd_rn(acc, a.shared[(size_t)t * a.d_model + row0 + r]);
        if (a.resid) acc = __fadd_rn(a.resid[(size_t)t * a.d_model + row0 + r], acc);
        if (a.accumulate) acc = __fadd_rn(o[r], acc);
        o[r] = acc;
    }
}

// ---------------------------------------------------------------------------
// Dequantiser through the same unit decoders (ggml dequantize_row_* float
// order).  One lane per unit; grid = ceil(total units / 256)
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(kThreads) void k_dequant(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                      int n_rows, int k) {
    extern __shared__ __align__(16) uint8_t smem[];
    if constexpr (QT == QT_IQ3_S) stage_iq3s_tables(smem);
    __syncthreads();
    const int NUS = units_per_row(QT, k);
    const long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= (long long)n_rows * NUS) return;
    const long long r = u / NUS;
    const int us = (int)(u % NUS);
    UnitWindow<QT> Wn;
    const uint8_t* row = src + (size_t)r * row_bytes(QT, k);
    Wn.load(row + (size_t)us * UnitFmt<QT>::BYTES, unit_len<QT>(k, us));
    unit_dequant<QT>(Wn, smem, dst + (size_t)r * k + (size_t)us * UnitFmt<QT>::ELEMS,
                     min(UnitFmt<QT>::ELEMS, k - us * UnitFmt<QT>::ELEMS));
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
    wg_quantize_row(x + (size_t)r * k, k, at, smem);   // blockDim.x == 256: sixteen row-slots
    __syncthreads();
    const ActLayout L(k, at);
    const int qb = block_elems(at), bb = block_bytes(at), nb = k / qb;
    uint8_t* yr = y + (size_t)r * nb * bb;
    const float* d = reinterpret_cast<const float*>(smem + L.off_d);
    for (int q = threadIdx.x; q < k; q += blockDim.x) {
        const int b = q / qb, j = q - b * qb;
        yr[(size_t)b * bb + (at == QT_Q8_K ? 4 : 2) + j] = smem[(q >> 8) * kActChunkStride + (q & 255)];
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
