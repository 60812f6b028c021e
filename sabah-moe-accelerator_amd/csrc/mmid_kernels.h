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

// Ids and pointer tables are read through the constant address space: they
// do not change during a kernel, and a workgroup-uniform read then becomes a
// scalar load, which has its own counter (waiting for it never waits for the
// vector loads issued before it).
typedef __attribute__((address_space(4))) const int32_t c_int32;
typedef __attribute__((address_space(4))) const uint64_t c_uint64;

// A wave-uniform value pinned to a scalar register.  (Values that went
// through a division or another vector op otherwise stay in vector registers,
// and so does everything computed from them.)
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// a wave-uniform pointer held in scalar registers
template <typename T>
__device__ inline T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ inline int read_id(const Routing& R, int t, int s) {
    return *(c_int32*)uniform_ptr(R.ids + (size_t)t * R.token_stride + (size_t)s * R.id_stride);
}

// expert matrix of (token t, slot s), or nullptr for an id outside [0, n_experts)
__device__ inline const uint8_t* expert_ptr(const ExpertSrc& E, const Routing& R, int t, int s, int n_slots) {
    if (E.ptrs) return reinterpret_cast<const uint8_t*>(*(c_uint64*)uniform_ptr(E.ptrs + (size_t)t * n_slots + s));
    const int e = R.ids ? read_id(R, t, s) : 0;
    if (e < 0 || e >= R.n_experts) return nullptr;
    return E.base + (size_t)e * E.expert_stride;
}

// The gate and up matrices of (token t, slot s): one id read serves both (or
// both table entries are requested before either is waited for)
__device__ inline void expert_pair(const ExpertSrc& G, const ExpertSrc& U, const Routing& R, int t, int s,
                                   int n_slots, const uint8_t*& g, const uint8_t*& u) {
    if (G.ptrs || U.ptrs) {
        g = expert_ptr(G, R, t, s, n_slots);
        u = expert_ptr(U, R, t, s, n_slots);
        return;
    }
    const int e = R.ids ? read_id(R, t, s) : 0;
    const bool ok = e >= 0 && e < R.n_experts;
    g = ok ? G.base + (size_t)e * G.expert_stride : nullptr;
    u = ok ? U.base + (size_t)e * U.expert_stride : nullptr;
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
// unit order, at contiguous bytes.  The workgroup walks them in passes of nv
// units per tile; a pass's tiles are staged in LDS, tile t at 16 * cpt * t,
// starting `lead` (its HBM address mod 16) bytes into its first 16-byte
// chunk, so staged bytes keep their HBM alignment mod 16.
//
// Loads: each tile has LPT = kThreads / n_mat lanes, and lane j of a tile
// reads the tile's chunks j, j + LPT, j + 2 LPT, ... - exactly StageIters
// of them (a static count, so waits for older loads stay exact): a lane past
// the tile's last chunk re-reads it, and lanes beyond n_mat * LPT re-read the
// last tile's chunks.  Consecutive lanes read consecutive chunks, so a load
// instruction of a wave reads up to 1 KB of contiguous HBM.  The load plan
// is a few integer operations per lane.  Once every lane has written its
// chunks to LDS and the workgroup has synchronised, lane g decodes units g,
// g + kThreads, ... of the pass (tile-major numbering).  The next pass's
// loads are issued before the current pass is decoded.
// ---------------------------------------------------------------------------
constexpr int kStageChunks = 2048;                            // 32 KB per workgroup
constexpr int kStageBytes = 16 * kStageChunks;
constexpr int kStageGuard = 16;
constexpr int kMaxTiles = 64;

// 16-byte loads per lane per pass
__host__ __device__ constexpr int stage_iters(int qt) {
    return qt == QT_IQ3_S ? 7 : qt == QT_Q4_K ? 10 : qt == QT_Q5_K ? 12 : qt == QT_Q6_K ? 14 : qt == QT_IQ3_XXS ? 7
         : (qt == QT_IQ4_NL || qt == QT_Q2_0) ? 5 : qt == QT_Q5_1 ? 7
         : qt == QT_IQ2_S ? 6 : 9;
}
// the same load count spread over nt threads
__host__ __device__ constexpr int stage_iters_nt(int qt, int nt) { return (stage_iters(qt) * kThreads + nt - 1) / nt; }
template <int QT, int NT = kThreads>
struct StageIters {
    static constexpr int V = stage_iters_nt(QT, NT);
};

// chunks of a tile of tile_bytes at any lead
__host__ __device__ inline int tile_chunks(int tile_bytes) { return (tile_bytes + 30) / 16; }
// chunks one tile may stage per pass: its share of the stage, and no more
// than its lanes load
__host__ __device__ inline int tile_chunk_cap(int qt, int n_mat) {
    return min(kStageChunks / n_mat, stage_iters(qt) * (kThreads / n_mat));
}
// passes of at most vmax units each, all of about the same size
__host__ __device__ inline int even_passes(int total, int vmax) {
    const int np = (total + vmax - 1) / vmax;
    return (total + np - 1) / np;
}
// the device forms of tile_chunk_cap / pass_units / even_passes: the same
// values through div_small (a generic integer division is some forty
// instructions on the kernels' critical path)
__device__ inline int tile_chunk_cap_d(int qt, int n_mat, int nt) {
    return min(div_small_u(kStageChunks, n_mat), stage_iters_nt(qt, nt) * div_small_u(nt, n_mat));
}
__device__ inline int even_passes_d(int total, int vmax) {
    const int np = div_small_u(total + vmax - 1, vmax);
    return div_small_u(total + np - 1, np);
}
// units per tile per pass: the largest V with tile_chunks(V * unit bytes) <= tile_chunk_cap
__host__ __device__ inline int pass_units(int qt, int n_mat, int unit_bytes) {
    return max(1, (16 * tile_chunk_cap(qt, n_mat) - 30) / unit_bytes);
}

// Q8_0, IQ4_NL (32-element blocks) and Q2_0 (64) rows need only be whole
// blocks: their units are four blocks, the last of a row 1..3
__host__ __device__ inline bool four_block_units(int qt) {
    return qt == QT_Q8_0 || qt == QT_Q5_1 || qt == QT_IQ4_NL || qt == QT_Q2_0;
}
__host__ __device__ inline int units_per_row(int qt, int k) {
    return four_block_units(qt) ? (k + 4 * block_elems(qt) - 1) / (4 * block_elems(qt)) : k / 256;
}
// fp32 terms of the row sum: one per block; one per 32 elements for IQ4_XS
// (its sub-blocks) and Q2_0 (its q8_0 activation blocks)
__host__ __device__ inline int contribs_per_row(int qt, int k) {
    return (qt == QT_IQ4_XS || qt == QT_Q2_0) ? k / 32 : k / block_elems(qt);
}
__host__ __device__ inline int unit_bytes(int qt) { return four_block_units(qt) ? 4 * (int)block_bytes(qt) : (int)block_bytes(qt); }

// Rows per workgroup: about one unit per lane, with the n_mat tiles staged in
// one pass where a row fits.
__host__ __device__ inline int rows_per_wg(int qt, int k, int n_mat) {
    const int nus = units_per_row(qt, k);
    const int by_lanes = kThreads / (n_mat * nus);
    const int by_stage = (16 * tile_chunk_cap(qt, n_mat) - 30) / (int)row_bytes(qt, k);
    return max(1, min(by_lanes, by_stage));
}

// ---------------------------------------------------------------------------
// LDS: static arrays hold what the decoder addresses with constant offsets
// (the IQ3_S tables, the staging area); dynamic LDS holds the activation rows
// and per-block partials:  [activations][partials]
// ---------------------------------------------------------------------------
struct Plan {
    int off_act, act_bytes, n_act, off_part, bytes;
};

__host__ __device__ inline int align16i(int v) { return (v + 15) & ~15; }

// n_act activation rows of k elements for weight type qt; part = n_part floats
__host__ __device__ inline Plan make_plan(int qt, int k, int n_act, int n_part) {
    Plan p{};
    p.off_act = 0;
    p.act_bytes = align16i((int)ActLayout(k, act_type(qt)).bytes);
    p.n_act = n_act;
    p.off_part = p.act_bytes * n_act;
    p.bytes = p.off_part + align16i(4 * n_part);
    return p;
}

// static LDS of a kernel instantiation: IQ3_S tables, the staged tiles'
// leads, then the staging area with a guard on each side
template <int QT>
struct StaticLds {
    static constexpr int TABLES = table_bytes(QT);
    static constexpr int LEADS = TABLES;
    static constexpr int STAGE = LEADS + 4 * kMaxTiles + kStageGuard;
    static constexpr int BYTES = STAGE + kStageBytes + kStageGuard;
};
// total LDS of a launch (static + dynamic), for the host's limit check
__host__ inline int launch_lds(int qt, const Plan& P) {
    const int tables = table_bytes(qt);
    return tables + 4 * kMaxTiles + 2 * kStageGuard + kStageBytes + P.bytes;
}

// bytes of unit us of a row of k elements
template <int QT>
__device__ inline int unit_len(int k, int us) {
    if constexpr (QT == QT_Q8_0 || QT == QT_Q5_1 || QT == QT_IQ4_NL || QT == QT_Q2_0)
        return block_bytes(QT) * min(4, k / block_elems(QT) - 4 * us);
    return UnitFmt<QT>::BYTES;
}

// dot of one unit (unit index us of its row) with activation row `act`; the
// unit's per-block contributions go to part_row
template <int QT>
__device__ inline void unit_into_part(const LdsWindow<QT>& Wn, const uint8_t* tabs, const uint8_t* act, int k, int us,
                                      float* part_row) {
    const ActLayout AL(k, act_type(QT));
    const float* dxa = reinterpret_cast<const float*>(act + AL.off_d);
    const int16_t* bsa = reinterpret_cast<const int16_t*>(act + AL.off_bsum);
    if constexpr (QT == QT_Q8_0 || QT == QT_IQ4_NL || QT == QT_Q5_1) {
        // Q5_1: the q8_1 s values ride in the bsum argument
        const int16_t* bs = QT == QT_Q5_1 ? reinterpret_cast<const int16_t*>(reinterpret_cast<const float*>(bsa) + 4 * us)
                                          : bsa;
        const uint8_t* chunk = act + (us >> 1) * kActChunkStride + (us & 1) * 128;
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, chunk, dxa + 4 * us, bs);
        const int nb = min(4, k / 32 - 4 * us);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j < nb) part_row[4 * us + j] = r.c[j];
    } else if constexpr (QT == QT_Q2_0) {
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, act + us * kActChunkStride, dxa + 8 * us, bsa);
        const int nc = 2 * min(4, k / 64 - 4 * us);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < nc) part_row[8 * us + j] = r.c[j];
    } else if constexpr (QT == QT_IQ4_XS) {
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, act + us * kActChunkStride, dxa + us, bsa + 16 * us);
#pragma unroll
        for (int j = 0; j < 8; ++j) part_row[8 * us + j] = r.c[j];
    } else {
        const uint8_t* chunk = act + us * kActChunkStride;
        const UnitDot<QT> r = unit_dot<QT>(Wn, tabs, chunk, dxa + us, bsa + 16 * us);
        part_row[us] = r.c[0];
    }
}

// the n block terms of a row summed in block order from zero (ggml's
// vec_dot); the loads of eight terms are issued before their adds
__device__ inline float row_sum(const float* part_row, int n) {
    float s = 0.0f;
    int b = 0;
    for (; b + 8 <= n; b += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = part_row[b + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) s = __fadd_rn(s, t[j]);
    }
    if (b < n) {                                            // the last 1..7 terms, also loaded first
        float t[7];
#pragma unroll
        for (int j = 0; j < 7; ++j) t[j] = b + j < n ? part_row[b + j] : 0.0f;
#pragma unroll
        for (int j = 0; j < 7; ++j)
            if (b + j < n) s = __fadd_rn(s, t[j]);
    }
    return s;
}

// acc + v[1] + v[2] + ... + v[n-1] in that order, v[i] = p[i * stride]: the
// loads of eight terms are issued before their adds, so the chain waits for
// LDS once per eight terms instead of once per term
__device__ inline float ordered_sum_from(float acc, const float* p, int stride, int n) {
    int i = 1;
    for (; i + 8 <= n; i += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = p[(i + j) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __fadd_rn(acc, t[j]);
    }
    for (; i < n; ++i) acc = __fadd_rn(acc, p[i * stride]);
    return acc;
}

// One workgroup's tiles.  Tile t is matrix tile_ptr(t) from its first row on
// (row0 already folded into the pointer): `nrows` rows of k elements at rb
// bytes, so its unit v = r * NUS + us sits at byte r * rb + us * unit bytes.
template <int QT, int NT = kThreads>
struct TileWalk {
    static constexpr int UB = UnitFmt<QT>::BYTES;
    int n_mat, NUS, NCB, total, V;
    size_t rb;
    float rcp_nus;
    __device__ TileWalk(int n_mat_, int nrows, size_t rb_, int k)
        : n_mat(uni(n_mat_)), NUS(uni(units_per_row(QT, k))), NCB(uni(contribs_per_row(QT, k))),
          total(uni(nrows * units_per_row(QT, k))),
          V(even_passes_d(total, max(1, (16 * tile_chunk_cap_d(QT, n_mat_, NT) - 30) / UB))), rb(rb_),
          rcp_nus(__builtin_amdgcn_rcpf((float)units_per_row(QT, k))) {}
    __device__ int byte_of(int v) const {
        const int r = div_small(v, rcp_nus);
        return (int)((size_t)r * rb) + (v - r * NUS) * UB;
    }
    // the same for a wave-uniform v, returned as a scalar
    __device__ int byte_of_u(int v) const {
        const int r = div_small_u(v, rcp_nus);
        return (int)((size_t)r * rb) + (v - r * NUS) * UB;
    }
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// one pass of the workgroup's tiles (NT threads)
template <int QT, int NT = kThreads>
struct TileRun {
    static constexpr int N = StageIters<QT, NT>::V;
    TileWalk<QT, NT> T;
    int v0, nv, cpt, b0, span;        // pass (uniform): first unit, units per tile, chunks per tile,
                                      // byte of unit v0, bytes of nv units
    int lpt, lt, lj;                  // lanes per tile; this lane's load tile and its index in it
    const uint8_t* src;               // this lane's load tile (the tile's first row)
    u32x4 d[N];
    int q[N];                         // chunk of each load, within the tile
    int lead;                         // the load tile's pass start address mod 16
};

template <int QT, int NT>
__device__ inline void set_pass(TileRun<QT, NT>& S, int v0) {
    S.v0 = v0;
    S.nv = uni(min(S.T.V, S.T.total - v0));
    S.b0 = S.T.byte_of_u(v0);
    S.span = uni(S.T.byte_of_u(v0 + S.nv) - S.b0);
    S.cpt = uni(tile_chunks(S.span));
}

template <int QT, int NT>
__device__ inline void pass_load(TileRun<QT, NT>& S) {
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    const uint8_t* P = S.src + S.b0;
    S.lead = (int)(reinterpret_cast<uintptr_t>(P) & 15);
    const uint8_t* g = P - S.lead;
    const int last = (S.lead + S.span - 1) >> 4;       // the tile's last chunk of the pass
#pragma unroll
    for (int it = 0; it < S.N; ++it) {
        S.q[it] = min(S.lj + S.lpt * it, last);
        S.d[it] = *(g_u32x4*)(g + 16 * S.q[it]);
    }
}

template <int QT, int NT>
__device__ inline void pass_store(const TileRun<QT, NT>& S, uint8_t* stage, int* leads) {
    uint8_t* dst = stage + 16 * S.cpt * S.lt;
#pragma unroll
    for (int it = 0; it < S.N; ++it) *reinterpret_cast<u32x4*>(dst + 16 * S.q[it]) = S.d[it];
    if (S.lj == 0) leads[S.lt] = S.lead;
}

// decode the pass's units, NT apart per lane (with 512 IQ3_S threads, a unit
// per lane pair: each lane sums half its items and the pair adds the two
// exact integer sums); contributions of unit (t, r, us) go to
// part + (t * part_rows + r) * NCB
template <int QT, int NT>
__device__ inline void pass_decode(const TileRun<QT, NT>& S, const uint8_t* tabs, const uint8_t* stage,
                                   const int* leads, int k, const uint8_t* act0, int act_stride, int part_rows,
                                   float* part) {
    constexpr bool SPLIT = (QT == QT_IQ3_S || QT == QT_Q4_K) && NT == 2 * kThreads;
    constexpr int PER = SPLIT ? 2 : 1;                  // lanes per unit
    const int n = S.T.n_mat * S.nv;
    const float rcp_nv = __builtin_amdgcn_rcpf((float)S.nv);
    // with two lanes per unit the halves sit 32 lanes apart (a half-wave's
    // field reads span 32 units): lane l of wave w takes unit 32 w + l % 32
    const int tid = (int)threadIdx.x;
    const int half = SPLIT ? (tid >> 5) & 1 : 0;
    const int u0 = SPLIT ? 32 * (tid >> 6) + (tid & 31) : tid;
    for (int u = u0; u < n; u += NT / PER) {           // both lanes of a pair iterate together
        const int t = div_small(u, rcp_nv);
        const int v = S.v0 + (u - t * S.nv);             // tile-relative unit (row-major over the rows)
        const int r = div_small(v, S.T.rcp_nus), us = v - r * S.T.NUS;
        const uint8_t* unit = stage + 16 * S.cpt * t + leads[t] + (int)((size_t)r * S.T.rb) + us * TileWalk<QT>::UB - S.b0;
        float* prow = part + (t * part_rows + r) * S.T.NCB;
        if constexpr (SPLIT && QT == QT_IQ3_S) {
            const uint8_t* act = act0 + t * act_stride;
            const ActLayout AL(k, QT_Q8_K);
            uint32_t G[UnitFmt<QT>::NF], A[4][8], dbits;
            iq3s_half_fields(unit, half, G, dbits);
            act_half(act + us * kActChunkStride, half, A);
            int bs = iq3s_half_bsum(G, tabs, A);
            bs += __shfl_xor(bs, 32);                    // the partner lane's half
            if (half == 0)
                prow[us] = __fmul_rn(__fmul_rn(h2f(dbits), reinterpret_cast<const float*>(act + AL.off_d)[us]), (float)bs);
        } else if constexpr (SPLIT) {                    // Q4_K: the halves' exact sums, then unit_dot's fp32 steps
            const uint8_t* act = act0 + t * act_stride;
            const ActLayout AL(k, QT_Q8_K);
            Q4kHalf Q;
            uint32_t A[4][8];
            q4k_half_fields(unit, half, Q);
            act_half(act + us * kActChunkStride, half, A);
            int isum, msum;
            q4k_half_sums(Q, half, A, reinterpret_cast<const int16_t*>(act + AL.off_bsum) + 16 * us, isum, msum);
            isum += __shfl_xor(isum, 32);
            msum += __shfl_xor(msum, 32);
            if (half == 0) {
                const float dx = reinterpret_cast<const float*>(act + AL.off_d)[us];
                const float d = h2f(Q.F[0]), dmin = h2f(Q.F[0] >> 16);
                prow[us] = __fsub_rn(__fmul_rn(__fmul_rn(d, dx), (float)isum), __fmul_rn(__fmul_rn(dmin, dx), (float)msum));
            }
        } else {
            LdsWindow<QT> Wn;
            Wn.load(unit);
            unit_into_part<QT>(Wn, tabs, act0 + t * act_stride, k, us, prow);
        }
    }
}

// Issue the first pass's loads.  tile_ptr(t) is the first row of tile t, for
// a per-lane t.  The caller issues its own prologue loads before this and
// waits for them after it (loads complete in order), then calls tiles_finish.
template <int QT, int NT, typename TilePtr>
__device__ inline void tiles_begin(TileRun<QT, NT>& S, TilePtr tile_ptr) {
    const int g = (int)threadIdx.x;
    S.lpt = div_small_u(NT, S.T.n_mat);
    const int lt = div_small(g, __builtin_amdgcn_rcpf((float)S.lpt));
    const bool idle = lt >= S.T.n_mat;
    S.lt = idle ? S.T.n_mat - 1 : lt;
    S.lj = idle ? S.lpt - 1 : g - lt * S.lpt;
    S.src = tile_ptr(S.lt);
    set_pass(S, 0);
    pass_load(S);
}

// Stage and decode every pass.  The workgroup barrier after the stores also
// publishes what the caller's prologue wrote to LDS (activations, tables);
// the one after each decode frees the stage and publishes the partials.
template <int QT, int NT>
__device__ inline void tiles_finish(TileRun<QT, NT>& S, const uint8_t* tabs, uint8_t* stage, int* leads, int k,
                                    const uint8_t* act0, int act_stride, int part_rows, float* part) {
    for (;;) {
        pass_store(S, stage, leads);
        __syncthreads();
        const TileRun<QT, NT> C = S;             // this pass (the registers of the next one are reused)
        const int next = C.v0 + C.nv;
        if (next < S.T.total) {
            set_pass(S, next);
            pass_load(S);
        }
        pass_decode(C, tabs, stage, leads, k, act0, act_stride, part_rows, part);
        __syncthreads();
        if (next >= S.T.total) break;
    }
}

// 64-bit value of lane `src` (0..63, per lane) of the wave
__device__ inline const uint8_t* lane_ptr(const uint8_t* p, int src) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

// activation rounds prefetched before the weights (more are loaded late)
constexpr int kRoundsX = 1;   // one row: 16 chunks of 256 (k <= 4096)
constexpr int kRoundsH = 2;   // slot rows: 32 chunk-rows (n_slots * ceil(d_ff / 256))

// ---------------------------------------------------------------------------
// MUL_MAT_ID (sabah_rt_mul_mat_id_v2 semantics, sabah_rt.cu:2791-2839):
//   dst[t][i][r] = W[ids[t][i]][r] . q8(x[t][i % x_rows])
// grid = (ceil(rows / R), n_ids, n_tokens).  Rows packed at row_stride form
// one tile; rows row_stride > row bytes apart are one tile each (R <= kMaxTiles).
// ---------------------------------------------------------------------------
// ggml_vec_sigmoid_f32: 1 / (1 + exp(-v))
__device__ inline float sigmoid_f32(float v) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v))); }

// Shared-expert gate logit w . x (qwen4exp.cpp:877-885, ffn_gate_inp_shexp
// times the layer input) in one fixed order:
// 256 strided partial sums (lane v sums elements v, v + 256, ... in turn),
// each wave of them summed by a butterfly (every lane ends with the same
// value), then the four wave sums in order.  The 256 threads of a workgroup
// call gate_dot_part, which stores each wave's sum in sums[wave]; after a
// barrier gate_dot_total gives every thread the logit.
__device__ inline void gate_dot_part(const float* w, const float* x, int n, float* sums) {
    const int v = (int)threadIdx.x;
    float p = 0.0f;
    for (int i = v; i < n; i += 256) p = __fadd_rn(p, __fmul_rn(w[i], x[i]));
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) p = __fadd_rn(p, __shfl_xor(p, m));
    if ((v & 63) == 0) sums[v >> 6] = p;
}
__device__ inline float gate_dot_total(const float* sums) {
    return __fadd_rn(__fadd_rn(__fadd_rn(sums[0], sums[1]), sums[2]), sums[3]);
}

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
    const float* sg_w;            // optional [sg_n] gate row: every output row of token t is scaled by
    const float* sg_x;            //   sigmoid(sg_w . sg_x[t]) (the shared expert's gate); sg_x [n_tokens][sg_n]
    int sg_n;
};

// The kernels' static LDS: IQ3_S tables (when QT is IQ3_S), the staged
// tiles' leads and the staging area.
#define SABAH_STATIC_LDS(QT)                                                              \
    __shared__ __align__(16) uint8_t lds_static[StaticLds<QT>::BYTES];                    \
    uint8_t* const tabs = lds_static;                                                    \
    int* const leads = reinterpret_cast<int*>(lds_static + StaticLds<QT>::LEADS);        \
    uint8_t* const stage = lds_static + StaticLds<QT>::STAGE;

// Waves per SIMD the tile kernels are compiled for.  Q6_K's fully unrolled unit
// decoder takes just over 256 registers (one wave per SIMD); bounded to two
// waves it fits in 256, which keeps a second workgroup's loads in flight.
__host__ __device__ constexpr int tile_min_waves(int qt) { return qt == QT_Q6_K ? 2 : 1; }

template <int QT>
__global__ __launch_bounds__(kThreads, tile_min_waves(QT)) void k_mmid(MmidArgs a) {
    SABAH_STATIC_LDS(QT)
    extern __shared__ __align__(16) uint8_t smem[];
    const int NCB = contribs_per_row(QT, a.k);
    const Plan P = make_plan(QT, a.k, 1, a.R * NCB);
    const int t = blockIdx.z, i = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.rows - row0);
    const size_t rb = row_bytes(QT, a.k);
    float* out = reinterpret_cast<float*>(a.dst + (size_t)t * a.dst_token_stride + (size_t)i * a.dst_id_stride) + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    const float* xr = reinterpret_cast<const float*>(a.x + (size_t)t * a.x_token_stride +
                                                     (size_t)(i % a.x_rows) * a.x_id_stride);
    // activation and table loads first, then the weights, so the prologue's
    // waits do not wait for the weights (loads complete in order); the expert
    // id is a scalar load with its own counter
    const ActBatch xb{xr, 0, 1, a.k, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    act_prefetch<kRoundsX, kThreads>(xb, xa);
    const TableRegs<QT, kThreads> gr = load_tables<QT, kThreads>((int)threadIdx.x);
    const uint8_t* w = expert_ptr(a.W, a.rt, t, i, a.n_ids);
    if (w == nullptr) {   // uniform across the workgroup
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += kThreads) out[r] = __builtin_nanf("");
        return;
    }
    w += (size_t)row0 * a.row_stride;
    const bool packed = a.row_stride == rb;
    auto tile_ptr = [&](int r) { return packed ? w : w + (size_t)r * a.row_stride; };
    TileRun<QT> S{TileWalk<QT>(packed ? 1 : nrows, packed ? nrows : 1, rb, a.k)};
    tiles_begin(S, tile_ptr);
    store_tables<QT, kThreads>(tabs, gr, (int)threadIdx.x);
    act_quantize<kRoundsX, kThreads>(xb, xa);
    // the gate's loads come after the weights', so it waits for what the
    // staging waits for anyway; the staging's barrier publishes the sums
    __shared__ float sg_sums[4];
    if (a.sg_w) gate_dot_part(a.sg_w, a.sg_x + (size_t)t * a.sg_n, a.sg_n, sg_sums);
    tiles_finish(S, tabs, stage, leads, a.k, act, 0, packed ? a.R : 1, part);
    const float sg = a.sg_w ? sigmoid_f32(gate_dot_total(sg_sums)) : 1.0f;
    for (int r = threadIdx.x; r < nrows; r += kThreads) {
        const float y = row_sum(part + r * NCB, NCB);
        out[r] = a.sg_w ? __fmul_rn(y, sg) : y;
    }
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

// h row r of a workgroup: a plain store, or (publish) an agent-scope store
// written through to memory, so a workgroup of the same grid on another XCD
// can read it once this one has waited for its stores and set its flag
__device__ inline void store_h(float* p, float v, bool publish) {
    if (publish) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// One workgroup of k_gate_up (kThreads threads): token t, slot s, rows
// row0 .. row0 + R of gate and up, h = silu(g) * u to hbase (laid out as
// a.h), published with store_h when `publish`.  tabs, leads, stage: the
// static LDS; smem: the plan's dynamic LDS.
template <int QT, int NT = kThreads>
__device__ inline void gate_up_tile(const GateUpArgs& a, int t, int s, int row0, uint8_t* tabs, int* leads,
                                    uint8_t* stage, uint8_t* smem, bool publish, float* hbase) {
    const int NCB = contribs_per_row(QT, a.d_model);
    const Plan P = make_plan(QT, a.d_model, 1, 2 * a.R * NCB);
    const int nrows = min(a.R, a.d_ff - row0);
    const size_t rb = row_bytes(QT, a.d_model);
    float* h = hbase + ((size_t)t * a.n_slots + s) * a.d_ff + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    const ActBatch xb{a.x + (size_t)t * a.d_model, 0, 1, a.d_model, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    act_prefetch<kRoundsX, NT>(xb, xa);
    const TableRegs<QT, NT> gr = load_tables<QT, NT>((int)threadIdx.x);
    const uint8_t *wg, *wu;
    expert_pair(a.G, a.U, a.rt, t, s, a.n_slots, wg, wu);
    if (wg == nullptr || wu == nullptr) {
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += NT) store_h(h + r, __builtin_nanf(""), publish);
        return;
    }
    wg += (size_t)row0 * rb;
    wu += (size_t)row0 * rb;
    auto tile_ptr = [&](int m) { return m ? wu : wg; };
    TileRun<QT, NT> S{TileWalk<QT, NT>(2, nrows, rb, a.d_model)};
    tiles_begin(S, tile_ptr);
    store_tables<QT, NT>(tabs, gr, (int)threadIdx.x);
    act_quantize<kRoundsX, NT>(xb, xa);
    tiles_finish(S, tabs, stage, leads, a.d_model, act, 0, a.R, part);
    for (int r = threadIdx.x; r < nrows; r += NT) {
        const float g = row_sum(part + r * NCB, NCB);
        const float up = row_sum(part + (a.R + r) * NCB, NCB);
        store_h(h + r, __fmul_rn(silu_f32(g), up), publish);
    }
}

// NT = 2 kThreads (Q4_K): two lanes per unit (pass_decode), twice the waves
template <int QT, int NT = kThreads>
__global__ __launch_bounds__(NT, tile_min_waves(QT)) void k_gate_up(GateUpArgs a) {
    SABAH_STATIC_LDS(QT)
    extern __shared__ __align__(16) uint8_t smem[];
    gate_up_tile<QT, NT>(a, blockIdx.z, blockIdx.y, blockIdx.x * a.R, tabs, leads, stage, smem, false, a.h);
}

// ---------------------------------------------------------------------------
// Gate/up + SwiGLU in rounds, for packed IQ3_S rows whose units per row
// divide 128.  R = 2 RR rows, RR = 128 / units per row: a workgroup owns R
// gate and R up rows, 256 units of each.  With PER = 2 two lanes share a unit
// (each sums half its items; DPP adds the pair's exact integer sums), so a
// wave owns 32 units of a round; with PER = 1 it owns 64.  Half the waves take
// the gate rows, half the up rows; a wave loads, stages and decodes its own
// contiguous units of each of its rounds, so it decodes as soon as its own
// bytes are in.  Round 0's loads are issued as soon as the ids are in; the
// later rounds' loads follow the prologue (table, q8 x), whose own loads
// would otherwise wait behind them in the memory pipeline (a chain of layers
// runs 1.8 % faster than with every round issued up front).  With 512
// threads a wave has two rounds and decodes round 0 while round 1 is in
// flight (1024 threads, one round per wave, needs 93 KB of LDS and ran no
// faster in a chain).  The staging regions (one per wave, reused by its
// rounds) are in dynamic LDS after the plan: 67 KB per workgroup with the
// tables.
// grid = (ceil(d_ff / R), n_slots, n_tokens)
// ---------------------------------------------------------------------------
// units of a round per wave
template <int PER>
struct RoundUnits {
    static constexpr int V = 64 / PER;
};
// 16-byte chunks of one wave's round at any lead, and the loads per lane that cover them
template <int QT, int PER>
struct WaveRoundChunks {
    static constexpr int V = (RoundUnits<PER>::V * UnitFmt<QT>::BYTES + 30) / 16;
    static constexpr int LOADS = (V + 63) / 64;
};
template <int QT, int NT, int PER>
struct GateUpRounds {
    static constexpr int NW = NT / 64;                      // waves
    static constexpr int WPM = NW / 2;                      // waves per matrix
    static constexpr int UPW = RoundUnits<PER>::V;          // units per wave and round
    static constexpr int RD = 256 / (WPM * UPW);            // rounds per wave
    static constexpr int WCH = WaveRoundChunks<QT, PER>::V;
    static constexpr int STAGE = NW * 16 * WCH;             // staging bytes
    static_assert(RD >= 1 && RD * WPM * UPW == 256, "a workgroup's 256 units per matrix split evenly");
};
__host__ __device__ inline bool gate_up_rounds_ok(int qt, int d_model) {
    const int nus = units_per_row(qt, d_model);
    return qt == QT_IQ3_S && d_model % 256 == 0 && nus <= 128 && 128 % nus == 0;
}
__host__ __device__ inline int rows_gate_up_rounds(int qt, int d_model) { return 256 / units_per_row(qt, d_model); }
constexpr int kGateUpRoundThreads = 2 * kThreads;
// dynamic LDS of a launch: the plan, then the staging regions
__host__ __device__ inline int gate_up_rounds_lds(const Plan& P, int stage) { return align16i(P.bytes) + stage; }

// One workgroup of k_gate_up_rounds: token t, slot s, rows row0 .. row0 + R.
// tabs: the IQ3_S table (kLdsTables bytes); smem: the plan's dynamic LDS;
// stage: the waves' staging regions (GateUpRounds::STAGE bytes).
template <int QT, int NT, int PER>
__device__ inline void gate_up_rounds_tile(const GateUpArgs& a, int t, int s, int row0, uint8_t* tabs, uint8_t* smem,
                                           uint8_t* stage, bool publish) {
    using GR = GateUpRounds<QT, NT, PER>;
    constexpr int UB = UnitFmt<QT>::BYTES;
    constexpr int UPW = GR::UPW, WPM = GR::WPM, RD = GR::RD;
    constexpr int WCH = GR::WCH, N = WaveRoundChunks<QT, PER>::LOADS;
    static_assert(PER == 1 || QT == QT_IQ3_S, "split units are IQ3_S only");
    const int NUS = units_per_row(QT, a.d_model), NCB = contribs_per_row(QT, a.d_model);
    const Plan P = make_plan(QT, a.d_model, 1, 2 * a.R * NCB);
    const int nrows = min(a.R, a.d_ff - row0);
    const size_t rb = row_bytes(QT, a.d_model);
    float* h = a.h + ((size_t)t * a.n_slots + s) * a.d_ff + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    const ActBatch xb{a.x + (size_t)t * a.d_model, 0, 1, a.d_model, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    act_prefetch<kRoundsX, NT>(xb, xa);
    GridRegs<NT> gr;
    if constexpr (QT == QT_IQ3_S) gr = load_grid_regs<NT>((int)threadIdx.x);
    const uint8_t *wg, *wu;
    expert_pair(a.G, a.U, a.rt, t, s, a.n_slots, wg, wu);
    if (wg == nullptr || wu == nullptr) {
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += NT) store_h(h + r, __builtin_nanf(""), publish);
        return;
    }
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63u);
    const int m = wave / WPM;
    const uint8_t* tile = (m ? wu : wg) + (size_t)row0 * rb;
    const int nvalid = nrows * NUS;                         // the tile's units in this workgroup
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    u32x4 d[RD][N];
    int q[RD][N], lead[RD], v0[RD];
    // round rd's loads: the wave's contiguous units, consecutive lanes on
    // consecutive 16-byte chunks
    auto issue_round = [&](int rd) {
        v0[rd] = WPM * UPW * rd + UPW * (wave % WPM);
        const int nu = min(UPW, nvalid - v0[rd]);
        const uint8_t* p = tile + (nu > 0 ? (size_t)v0[rd] * UB : 0);
        lead[rd] = (int)(reinterpret_cast<uintptr_t>(p) & 15);
        const uint8_t* g = p - lead[rd];
        const int last = nu > 0 ? (lead[rd] + nu * UB - 1) >> 4 : 0;
#pragma unroll
        for (int it = 0; it < N; ++it) {
            q[rd][it] = min(lane + 64 * it, last);
            d[rd][it] = *(g_u32x4*)(g + 16 * q[rd][it]);
        }
    };
    issue_round(0);
    if constexpr (QT == QT_IQ3_S) store_iq3s_tables<NT>(tabs, gr, (int)threadIdx.x);
    act_quantize<kRoundsX, NT>(xb, xa);
#pragma unroll
    for (int rd = 1; rd < RD; ++rd) issue_round(rd);
    __syncthreads();                                        // activations and tables ready
    uint8_t* region = stage + 16 * WCH * wave;
    const float rcp_nus = __builtin_amdgcn_rcpf((float)NUS);
    // the lane's unit in the round and its half: with two lanes per unit, the
    // halves sit 32 lanes apart, so a half-wave's field reads come from 32
    // units (110 bytes apart) rather than 16 units twice, on fewer shared banks
    const int j = PER == 2 ? lane & 31 : lane, half = PER == 2 ? lane >> 5 : 0;
    // a lane's unit column is the same in every round (a wave's rounds are
    // 128 units apart and NUS divides 128), so its activation half is read once
    uint32_t A[4][8];
    if constexpr (PER == 2) {
        const int vj = v0[0] + j;
        act_half(act + (vj - div_small(vj, rcp_nus) * NUS) * kActChunkStride, half, A);
    }
#pragma unroll
    for (int rd = 0; rd < RD; ++rd) {
        // the wave's own chunks: LDS operations of one wave complete in order,
        // so its reads below see these writes, and round 1's writes come after
        // round 0's reads
#pragma unroll
        for (int it = 0; it < N; ++it) *reinterpret_cast<u32x4*>(region + 16 * q[rd][it]) = d[rd][it];
        if (j < nvalid - v0[rd]) {                          // both lanes of a pair alike
            const int v = v0[rd] + j;
            const int r = div_small(v, rcp_nus), us = v - r * NUS;
            const uint8_t* unit = region + lead[rd] + j * UB;
            float* prow = part + (m * a.R + r) * NCB;
            if constexpr (PER == 2) {
                const ActLayout AL(a.d_model, QT_Q8_K);
                uint32_t G[UnitFmt<QT>::NF], dbits;
                iq3s_half_fields(unit, half, G, dbits);
                int bs = iq3s_half_bsum(G, tabs, A);
                bs += __shfl_xor(bs, 32);                  // the partner lane's half
                if (half == 0)
                    prow[us] = __fmul_rn(__fmul_rn(h2f(dbits), reinterpret_cast<const float*>(act + AL.off_d)[us]),
                                         (float)bs);
            } else {
                LdsWindow<QT> Wn;
                Wn.load(unit);
                unit_into_part<QT>(Wn, tabs, act, a.d_model, us, prow);
            }
        }
    }
    __syncthreads();                                        // partials complete
    for (int r = threadIdx.x; r < nrows; r += NT) {
        const float g = row_sum(part + r * NCB, NCB);
        const float up = row_sum(part + (a.R + r) * NCB, NCB);
        store_h(h + r, __fmul_rn(silu_f32(g), up), publish);
    }
}

template <int QT, int NT, int PER = 2>
__global__ __launch_bounds__(NT) void k_gate_up_rounds(GateUpArgs a) {
    __shared__ __align__(16) uint8_t tabs[QT == QT_IQ3_S ? kLdsTables : 16];
    extern __shared__ __align__(16) uint8_t smem[];
    const Plan P = make_plan(QT, a.d_model, 1, 2 * a.R * contribs_per_row(QT, a.d_model));
    gate_up_rounds_tile<QT, NT, PER>(a, blockIdx.z, blockIdx.y, blockIdx.x * a.R, tabs, smem, smem + align16i(P.bytes),
                                     false);
}

// ---------------------------------------------------------------------------
// MUL_MAT_ID of IQ3_S slots in per-wave rounds: k_gate_up_rounds' scheme for
// the one matrix of a drop-in call (llama.cpp's gate, up and down nodes at
// decode, or a few tokens' while their row tiles stay single-pass; more tokens
// take k_mmid's grown tiles or the grouped kernels).  A workgroup of
// kMmidRoundThreads threads takes R = 256 /
// (units per row) packed rows of the slot's matrix, at most 256 units; each of
// its eight waves owns 32 consecutive units (its contiguous bytes), issues
// their loads as soon as the expert id is in, stages them in a private LDS
// region and decodes them, two lanes per unit, without waiting for the other
// waves; x is quantised while the loads fly.  k_mmid instead stages the whole
// tile behind one barrier, one lane per unit.  The integer unit sums and the
// fp32 steps are k_mmid's (and the row sums row_sum's), so the results are
// bit-identical to it.
// grid = (ceil(rows / R), n_ids, n_tokens)
// ---------------------------------------------------------------------------
constexpr int kMmidRoundThreads = 2 * kThreads;
// static LDS of k_mmid_rounds: the codebook table and the guarded staging regions
constexpr int kMmidRoundStaticLds = kLdsTables + 32 + (kMmidRoundThreads / 64) * 16 * WaveRoundChunks<QT_IQ3_S, 2>::V;
__host__ __device__ inline int rows_mmid_rounds(int qt, int k) { return 256 / units_per_row(qt, k); }
// the calls it serves: IQ3_S, packed rows of whole 256-element units, no gate row
__host__ __device__ inline bool mmid_rounds_ok(int qt, int k, size_t row_stride, bool gated) {
    return qt == QT_IQ3_S && k % 256 == 0 && k <= 256 * 256 && row_stride == row_bytes(qt, k) && !gated;
}

template <int NT>
__global__ __launch_bounds__(NT) void k_mmid_rounds(MmidArgs a) {
    constexpr int QT = QT_IQ3_S, PER = 2;
    constexpr int UB = UnitFmt<QT>::BYTES, UPW = RoundUnits<PER>::V, NW = NT / 64;
    constexpr int WCH = WaveRoundChunks<QT, PER>::V, N = WaveRoundChunks<QT, PER>::LOADS;
    static_assert(NW * UPW == 256, "a workgroup's waves cover its 256 units in one round");
    __shared__ __align__(16) uint8_t tabs[kLdsTables];
    // the waves' staging regions, with a guard on each side: a unit's field
    // reads start two bytes before it and end four bytes past it (never used)
    __shared__ __align__(16) uint8_t stage_mem[16 + NW * 16 * WCH + 16];
    static_assert(kLdsTables + sizeof(stage_mem) == kMmidRoundStaticLds, "static LDS as the host counts it");
    extern __shared__ __align__(16) uint8_t smem[];
    const int NUS = units_per_row(QT, a.k), NCB = contribs_per_row(QT, a.k);
    const Plan P = make_plan(QT, a.k, 1, a.R * NCB);
    const int t = blockIdx.z, i = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.rows - row0);
    const size_t rb = row_bytes(QT, a.k);
    float* out = reinterpret_cast<float*>(a.dst + (size_t)t * a.dst_token_stride + (size_t)i * a.dst_id_stride) + row0;
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    const float* xr = reinterpret_cast<const float*>(a.x + (size_t)t * a.x_token_stride +
                                                     (size_t)(i % a.x_rows) * a.x_id_stride);
    const ActBatch xb{xr, 0, 1, a.k, act_type(QT), act, 0};
    ActRegs<kRoundsX> xa;
    act_prefetch<kRoundsX, NT>(xb, xa);
    const GridRegs<NT> gr = load_grid_regs<NT>((int)threadIdx.x);
    const uint8_t* w = expert_ptr(a.W, a.rt, t, i, a.n_ids);
    if (w == nullptr) {   // uniform across the workgroup
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += NT) out[r] = __builtin_nanf("");
        return;
    }
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = (int)(threadIdx.x & 63u);
    // the wave's units v0 .. v0 + nu (none for a wave past a short last tile):
    // consecutive lanes load consecutive 16-byte chunks of their bytes
    const int v0 = UPW * wave, nu = min(UPW, nrows * NUS - v0);
    const uint8_t* p = w + (size_t)row0 * rb + (nu > 0 ? (size_t)v0 * UB : 0);
    const int lead = (int)(reinterpret_cast<uintptr_t>(p) & 15);
    const uint8_t* g = p - lead;
    const int last = nu > 0 ? (lead + nu * UB - 1) >> 4 : 0;
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    u32x4 d[N];
    int q[N];
#pragma unroll
    for (int it = 0; it < N; ++it) {
        q[it] = min(lane + 64 * it, last);
        d[it] = *(g_u32x4*)(g + 16 * q[it]);
    }
    store_iq3s_tables<NT>(tabs, gr, (int)threadIdx.x);
    act_quantize<kRoundsX, NT>(xb, xa);
    __syncthreads();                                        // activations and table ready
    // the wave's own chunks: LDS operations of one wave complete in order, so
    // its reads below see these writes
    uint8_t* region = stage_mem + 16 + 16 * WCH * wave;
#pragma unroll
    for (int it = 0; it < N; ++it) *reinterpret_cast<u32x4*>(region + 16 * q[it]) = d[it];
    // two lanes per unit, its halves 32 lanes apart (a half-wave's field reads
    // then come from 32 units rather than 16 units twice)
    const int j = lane & 31, half = lane >> 5;
    if (j < nu) {                                           // both lanes of a pair alike
        const int v = v0 + j;
        const int r = div_small(v, __builtin_amdgcn_rcpf((float)NUS)), us = v - r * NUS;
        uint32_t A[4][8];
        act_half(act + us * kActChunkStride, half, A);
        uint32_t G[UnitFmt<QT>::NF], dbits;
        iq3s_half_fields(region + lead + j * UB, half, G, dbits);
        int bs = iq3s_half_bsum(G, tabs, A);
        bs += __shfl_xor(bs, 32);                          // the partner lane's half
        if (half == 0) {
            const ActLayout AL(a.k, QT_Q8_K);
            part[r * NCB + us] =
                __fmul_rn(__fmul_rn(h2f(dbits), reinterpret_cast<const float*>(act + AL.off_d)[us]), (float)bs);
        }
    }
    __syncthreads();                                        // partials complete
    for (int r = threadIdx.x; r < nrows; r += NT) out[r] = row_sum(part + r * NCB, NCB);
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
    // optional: h already quantised, one activation row (the kernels' layout,
    // kDownHqRow(qt, d_ff) bytes) per (token, slot), token-major
    const uint8_t* hq;
};

// Bytes of one pre-quantised h row, and the most a workgroup copies in: with
// several tokens per launch, h is quantised once per (token, slot) row by a
// k_quant_rows launch instead of once per row tile by every workgroup.
__host__ __device__ inline int down_hq_row_bytes(int qt, int d_ff) { return align16i((int)ActLayout(d_ff, act_type(qt)).bytes); }
constexpr int kDownHqLoads = 4;                            // 16-byte loads per lane per 256 threads
__host__ __device__ inline bool down_hq_fits(int qt, int d_ff, int n_slots) {
    return n_slots * down_hq_row_bytes(qt, d_ff) <= 16 * kDownHqLoads * kThreads;
}

template <int QT, int NT = kThreads, bool HQ = false>
__global__ __launch_bounds__(NT, tile_min_waves(QT)) void k_down_combine(DownArgs a) {
    constexpr int RH = NT == kThreads ? kRoundsH : 1;      // activation rounds prefetched
    constexpr int HQN = kDownHqLoads * kThreads / NT;
    SABAH_STATIC_LDS(QT)
    extern __shared__ __align__(16) uint8_t smem[];
    const int NCB = contribs_per_row(QT, a.d_ff);
    const Plan P = make_plan(QT, a.d_ff, a.n_slots, a.n_slots * a.R * NCB);
    const int t = blockIdx.y, row0 = blockIdx.x * a.R;
    const int nrows = min(a.R, a.d_model - row0);
    const size_t rb = row_bytes(QT, a.d_ff);
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    // lane s of every wave holds slot s's tile (lanes past n_slots repeat the
    // last slot); a slot with an invalid id stages expert 0's rows, never
    // used: the output is poisoned.  The id loads go first, so waiting for
    // them does not wait for the activation loads.
    const int lane = (int)(threadIdx.x & 63u);
    const SlotWord sw = load_slot_word(a.D, a.rt, t, min(lane, a.n_slots - 1), a.n_slots);
    __builtin_amdgcn_sched_barrier(0);
    const ActBatch hb{a.h + (size_t)t * a.n_slots * a.d_ff, (size_t)a.d_ff, a.n_slots, a.d_ff, act_type(QT), act,
                      P.act_bytes};
    ActRegs<RH> ha;
    u32x4 hqv[HQ ? HQN : 1];
    const int hq_chunks = HQ ? (a.n_slots * P.act_bytes) >> 4 : 0;
    if constexpr (HQ) {        // the token's q8 h rows, as 16-byte chunks (every lane loads HQN)
        const u32x4* src = reinterpret_cast<const u32x4*>(a.hq + (size_t)t * a.n_slots * P.act_bytes);
#pragma unroll
        for (int i = 0; i < HQN; ++i) hqv[i] = src[min((int)threadIdx.x + NT * i, hq_chunks - 1)];
    } else {
        act_prefetch<RH, NT>(hb, ha);
    }
    // the epilogue's own inputs (router weight of this thread's first
    // (slot, row) and this thread's row of shared / resid / out) are read now,
    // so their latency hides behind the expert loads -- except in Q6_K's
    // q8-h form, where the four registers held across the decode loop spill
    // (the epilogue then reads them itself)
    constexpr bool EARLY = !(QT == QT_Q6_K && HQ);
    const float* wt = a.w + (size_t)t * a.n_slots;
    const float rcp_r = __builtin_amdgcn_rcpf((float)a.R);
    const int i0 = (int)threadIdx.x, r0 = (int)threadIdx.x;
    const size_t orow = (size_t)t * a.d_model + row0 + r0;
    float w0 = 0.0f, sh0 = 0.0f, rs0 = 0.0f, ac0 = 0.0f;
    if constexpr (EARLY) {
        w0 = i0 < a.n_slots * a.R ? wt[div_small(i0, rcp_r)] : 0.0f;
        sh0 = a.shared && r0 < nrows ? a.shared[orow] : 0.0f;
        rs0 = a.resid && r0 < nrows ? a.resid[orow] : 0.0f;
        ac0 = a.accumulate && r0 < nrows ? a.out[orow] : 0.0f;
    }
    const TableRegs<QT, NT> gr = load_tables<QT, NT>((int)threadIdx.x);
    const uint8_t* e = resolve_slot_word(a.D, a.rt, sw);
    const bool bad = __any(e == nullptr);
    const uint8_t* mine = (e ? e : a.D.base) + (size_t)row0 * rb;
    auto tile_ptr = [&](int m) { return lane_ptr(mine, m); };
    TileRun<QT, NT> S{TileWalk<QT, NT>(a.n_slots, nrows, rb, a.d_ff)};
    tiles_begin(S, tile_ptr);
    store_tables<QT, NT>(tabs, gr, (int)threadIdx.x);
    if constexpr (HQ) {
#pragma unroll
        for (int i = 0; i < HQN; ++i)
            if ((int)threadIdx.x + NT * i < hq_chunks) reinterpret_cast<u32x4*>(act)[threadIdx.x + NT * i] = hqv[i];
    } else {
        act_quantize<RH, NT>(hb, ha);
    }
    tiles_finish(S, tabs, stage, leads, a.d_ff, act, P.act_bytes, a.R, part);
    float* o = a.out + (size_t)t * a.d_model + row0;
    if (bad) {
        flag_error(a.err);
        for (int r = threadIdx.x; r < nrows; r += NT) o[r] = __builtin_nanf("");
        return;
    }
    // y_s[r] * w_s of every (slot, row) in parallel, kept in the row's first partial
    for (int i = i0; i < a.n_slots * a.R; i += NT) {
        const int sl = div_small(i, rcp_r);
        if (i - sl * a.R < nrows)
            part[i * NCB] = __fmul_rn(row_sum(part + i * NCB, NCB), EARLY && i == i0 ? w0 : wt[sl]);
    }
    __syncthreads();
    for (int r = r0; r < nrows; r += NT) {
        const size_t q = (size_t)t * a.d_model + row0 + r;
        const bool first = EARLY && r == r0;
        float acc = ordered_sum_from(part[r * NCB], part + r * NCB, a.R * NCB, a.n_slots);
        if (a.shared) acc = __fadd_rn(acc, first ? sh0 : a.shared[q]);
        if (a.resid) acc = __fadd_rn(first ? rs0 : a.resid[q], acc);
        if (a.accumulate) acc = __fadd_rn(first ? ac0 : o[r], acc);
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
    store_tables<QT, kThreads>(smem, load_tables<QT, kThreads>((int)threadIdx.x), (int)threadIdx.x);
    __syncthreads();
    const int NUS = units_per_row(QT, k);
    const long long u = (long long)blockIdx.x * kThreads + threadIdx.x;
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
// ggml's own block layout (block_q8_0: fp16 d + 32 int8; block_q8_1: fp16 d,
// fp16 s + 32 int8; block_q8_K: f32 d + 256 int8 + 16 int16 bsums).
// grid = n_rows, one workgroup per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_quantize_act_ggml(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                                int k, int at) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int r = blockIdx.x;
    wg_quantize_row(x + (size_t)r * k, k, at, smem);   // 256 threads: sixteen row-slots
    __syncthreads();
    const ActLayout L(k, at);
    const int qb = block_elems(at), bb = block_bytes(at), nb = k / qb;
    uint8_t* yr = y + (size_t)r * nb * bb;
    const float* d = reinterpret_cast<const float*>(smem + L.off_d);
    for (int q = threadIdx.x; q < k; q += kThreads) {
        const int b = q / qb, j = q - b * qb;
        yr[(size_t)b * bb + (at == QT_Q8_K ? 4 : at == QT_Q8_1 ? 4 : 2) + j] = smem[(q >> 8) * kActChunkStride + (q & 255)];
    }
    for (int b = threadIdx.x; b < nb; b += kThreads) {
        if (at == QT_Q8_K) {
            const float dv = d[b];
            memcpy(yr + (size_t)b * bb, &dv, 4);
            const int16_t* bs = reinterpret_cast<const int16_t*>(smem + L.off_bsum) + 16 * b;
            memcpy(yr + (size_t)b * bb + 260, bs, 32);
        } else {
            const unsigned short hb = __half_as_ushort(__float2half_rn(d[b]));
            yr[(size_t)b * bb] = (uint8_t)(hb & 0xff);
            yr[(size_t)b * bb + 1] = (uint8_t)(hb >> 8);
            if (at == QT_Q8_1) {                        // s, already fp16-rounded
                const float sv = reinterpret_cast<const float*>(smem + L.off_bsum)[b];
                const unsigned short hs = __half_as_ushort(__float2half_rn(sv));
                yr[(size_t)b * bb + 2] = (uint8_t)(hs & 0xff);
                yr[(size_t)b * bb + 3] = (uint8_t)(hs >> 8);
            }
        }
    }
}

}  // namespace sabah
