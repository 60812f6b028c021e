// One launch per MoE layer at one token (IQ3_S gate, up and down): the
// gate/up + SwiGLU workgroups and the down + combine workgroups run in the
// same grid, so the down weights stream from HBM while gate/up decodes.
//
// The layer is the one the two-kernel form computes (k_gate_up_rounds, then
// k_down_combine: ggml's MUL_MAT_ID + GLU, MUL_MAT_ID on h, the slot-ordered
// weighted sum; qwen4exp.cpp:848-862, sabah_rt.cu:2725-2785), with the same
// unit decoders, integer sums and fp32 steps in the same order, so the
// results are bit-identical to it.
//
// Grid: n_g gate/up workgroups (ids 0 .. n_g-1), then n_d down workgroups.
// Workgroups are dispatched in id order, so every gate/up workgroup has been
// dispatched before any down workgroup: a down workgroup waits only for
// workgroups that are running or done, and gate/up workgroups wait for
// nothing.  Every wait is also bounded (kLayerIdleTicks without progress):
// one that runs out poisons its rows, sets the sticky error word to 2 and
// ends, so every wave of the grid exits.
//
// The h handoff, per workgroup and without shared counters:
//   gate/up: h rows stored write-through to memory (agent-scope stores), the
//     stores waited for, then its flag sync[g] set (an agent-scope store);
//   down: a head start of d_delay left to the gate/up weight loads, then
//     the codebook table built, the weights loaded and staged in LDS,
//     and each lane's half unit decoded to int8 in registers, all while
//     gate/up runs; then wave 0 waits for the flags, h is read with ordinary
//     loads, quantised, and dotted with the decoded weights.  One down
//     workgroup per XCD (its leader) polls the n_g flags with agent-scope
//     loads (16 bytes per lane per poll) and then stores its XCD's flag,
//     which the XCD's other down workgroups poll, one word each, so the
//     gate/up workgroups' stores do not queue behind 256 pollers of the same
//     lines.  The XCD is the hardware's XCC_ID register.  The leader is
//     elected on the device: each down workgroup, on arrival, swaps this
//     launch's number into its XCD's ticket, and the one that gets back a
//     different number (the previous launch's) leads.  So every XCD that runs
//     a down workgroup has exactly one leader, wherever the dispatcher
//     places the workgroups (all on one XCD, some XCDs without any).  An
//     XCD's L2 and a CU's L1 start each launch without lines of h
//     (kernel-boundary coherence of device memory), and no workgroup reads
//     h before the flags, so the first read of a line on an XCD fetches it
//     from memory and the XCD's other down workgroups hit the line in L2.
// Forward progress needs no co-residency: down workgroups wait only for
// gate/up workgroups, which were all dispatched before the first down
// workgroup and wait for nothing; a follower waits only for its XCD's leader,
// which is already running (it took the ticket).  The waits are bounded by
// time without progress, not by total time: a leader's clock restarts
// whenever more gate/up flags are set, and a follower's whenever its leader
// reports a higher count, so a layer that is slowed (time-sliced with other
// work, CUs held by another stream's kernel) still completes; only a wait
// that sees no progress for kLayerIdleTicks gives up.
// Flags never go back to zero: every entry of sync (kSyncG flags, then
// kSyncD down counters) advances by one per launch.  A workgroup reads its
// own entry at start (the number of launches so far, n) and waits for or
// writes n + 1; down workgroup 0 advances the entries this launch does not
// use.  So a HIP graph can replay the kernel with unchanged arguments.
#pragma once
#include "mmid_kernels.h"

namespace sabah {

// Layout in 32-bit words: kSyncG gate/up flags (dense, polled 16 bytes per
// lane), kSyncD down counters (each read and written only by its owner, at
// its start and end), kSyncXcds per-XCD flags (one 128-byte line each:
// word 0 the launch number once the XCD's leader saw every gate/up flag,
// word 1 the count of flags the leader has seen so far), kSyncXcds per-XCD
// leader tickets (one line each, touched only by the XCD's own workgroups).
// (Gate/up flags one per line, written whole, measured slower: the pollers
// then read 240 lines per poll.)
constexpr int kLine = 32;                               // words per 128-byte line
constexpr int kSyncG = 1024, kSyncD = 1024, kSyncXcds = 8;
constexpr int kSyncDOff = kSyncG;
constexpr int kSyncX = kSyncDOff + kSyncD;              // first per-XCD flag (line aligned)
constexpr int kSyncT = kSyncX + kSyncXcds * kLine;      // first per-XCD leader ticket
constexpr int kSyncWords = kSyncT + kSyncXcds * kLine;
// A wait gives up after this long without progress: 50 ms of s_memrealtime
// (100 MHz).  It guards against a hang, not against a slow layer (one layer
// takes about 12 us).
constexpr unsigned long long kLayerIdleTicks = 5000000;
constexpr unsigned kErrLayerWait = 2u;                  // sticky error word: a down workgroup's wait ran out
constexpr int kLayerThreads = 512;

struct LayerArgs {
    GateUpArgs gu;              // gate/up workgroups: h of token 0
    DownArgs dn;                // down workgroups
    int n_g, g_tiles;           // gate/up workgroups (g_tiles row tiles per slot)
    int n_d;                    // down workgroups
    uint32_t* sync;             // [kSyncWords] lockstep flags (layout above)
    uint32_t wait_skew;         // 0; a test of the timeout path sets 1: the down workgroups wait for a
                                // flag value no gate/up workgroup writes, so their bounded wait runs out
    uint32_t d_delay;           // s_memrealtime ticks (10 ns) the down workgroups wait before their loads
    uint32_t idle_ticks;        // kLayerIdleTicks; the timeout test shortens it
    int xcd_groups;             // 0: down workgroups grouped by their hardware XCD; g > 0 (a placement
                                // test): grouped as if down workgroup j ran on XCD j % g, so every
                                // grouping the dispatcher could produce (all on one XCD, XCDs left
                                // empty) can be exercised; the XCD flag is then stored at agent scope,
                                // since a group's members sit on different XCDs
};

// LDS of the fused kernel: the down role's static layout (IQ3_S table, tile
// leads, staging area; the gate/up role stages its rounds in the same area),
// dynamic: the larger of the two roles' plans
__host__ __device__ inline int layer_dyn_lds(const GateUpArgs& gu, const DownArgs& dn) {
    const Plan Pg = make_plan(QT_IQ3_S, gu.d_model, 1, 2 * gu.R * contribs_per_row(QT_IQ3_S, gu.d_model));
    const Plan Pd = make_plan(QT_IQ3_S, dn.d_ff, dn.n_slots, dn.n_slots * dn.R * contribs_per_row(QT_IQ3_S, dn.d_ff));
    return max(Pg.bytes, Pd.bytes);
}

__device__ inline unsigned long long wall_ticks() { return __builtin_amdgcn_s_memrealtime(); }

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

__device__ inline unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & (unsigned)(kSyncXcds - 1);
}

// Wave 0 of a follower waits until word 0 of its XCD's flag line holds
// `target` (agent-scope loads of words 0 and 1).  The clock restarts whenever
// word 1, the leader's count of flags seen, changes.
__device__ inline bool wait_line(const uint32_t* line, uint32_t target, unsigned long long idle) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(line), (short)0, 8, 0x00020000);
    unsigned long long t0 = wall_ticks();
    uint32_t seen = ~0u;
    for (;;) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, 0, 0, 16);
        const uint32_t flag = (uint32_t)__builtin_amdgcn_readfirstlane((int)v[0]);
        const uint32_t count = (uint32_t)__builtin_amdgcn_readfirstlane((int)v[1]);
        if (flag == target) return true;
        const unsigned long long now = wall_ticks();
        if (count != seen) {
            seen = count;
            t0 = now;
        } else if (now - t0 > idle) {
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave 0 of a leader waits until the gate/up flags [0, n) all hold `target`;
// true when they do, false when a wait saw no new flag for `idle` ticks.  One
// 16-byte agent-scope load per lane per poll covers 256 flags (loads past n
// return 0 and are masked).  Whenever the number of set flags rises, the
// clock restarts and lane 0 stores the number in word 1 of `line`, the
// followers' progress word.
__device__ inline bool wait_flags(const uint32_t* sync, int n, uint32_t target, uint32_t* line,
                                  unsigned long long idle) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(sync), (short)0, n * 4, 0x00020000);
    const int lane = (int)(threadIdx.x & 63u);
    unsigned long long t0 = wall_ticks();
    int best = -1;
    for (;;) {
        int set = 0;
        for (int base = 0; base < n; base += 256) {
            const int f = base + 4 * lane;
            if (f < n) {
                const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(rs, f * 4, 0, 16);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (f + j < n && v[j] == target) ++set;
            }
        }
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) set += __shfl_xor(set, m);
        set = __builtin_amdgcn_readfirstlane(set);
        if (set == n) return true;
        const unsigned long long now = wall_ticks();
        if (set > best) {
            best = set;
            t0 = now;
            if (lane == 0) __hip_atomic_store(line + 1, (uint32_t)set, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (now - t0 > idle) {
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

// a whole 128-byte flag line set to v by the first 32 lanes of wave 0 (one
// ordinary store instruction).  The line stays in this XCD's L2, and the
// XCD's agent-scope polls (wait_line) see it there at once: an agent-scope
// load returns a line its L2 holds modified (measured on MI355X: a plain
// store seen by the sc1 polls of every CU of its XCD before the store's own
// completion returned to the writer, and by no CU of another XCD).
__device__ inline void store_flag_line(uint32_t* line, uint32_t v) {
    if (threadIdx.x < kLine) line[threadIdx.x] = v;
}

// Wave 0 of a down workgroup waits for h: its XCD's leader (whose ticket
// swap returned another launch's number) for every gate/up flag, then sets
// the XCD's flag; a follower for that flag.  True once h is complete, false
// when the wait ran out.
__device__ inline bool layer_wait_h(const LayerArgs& a, uint32_t target, unsigned x, uint32_t ticket) {
    uint32_t* xf = a.sync + kSyncX + kLine * x;
    if ((uint32_t)__builtin_amdgcn_readfirstlane((int)ticket) != target) {   // this XCD's leader
        const bool done = wait_flags(a.sync, a.n_g, target + a.wait_skew, xf, a.idle_ticks);
        if (done) {
            if (a.xcd_groups) {
                if (threadIdx.x == 0) __hip_atomic_store(xf, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                store_flag_line(xf, target);
            }
        }
        return done;
    }
    return wait_line(xf, target + a.wait_skew, a.idle_ticks);
}

// The down workgroups' epilogue (k_down_combine's order): y_s[r] * w_s of
// every (slot, row) in parallel, kept in the row's first partial, then each
// row's slot-ordered sum, shared row, residual and accumulator.  w0, sh0,
// rs0, ac0: this thread's prefetched router weight and row values.
__device__ inline void layer_combine(const DownArgs& d, int NCB, int nrows, float* part, float* o, size_t row0,
                                     float w0, float sh0, float rs0, float ac0, int NT) {
    const float rcp_r = __builtin_amdgcn_rcpf((float)d.R);
    const int i0 = (int)threadIdx.x, r0 = (int)threadIdx.x;
    for (int i = i0; i < d.n_slots * d.R; i += NT) {
        const int sl = div_small(i, rcp_r);
        if (i - sl * d.R < nrows) part[i * NCB] = __fmul_rn(row_sum(part + i * NCB, NCB), i == i0 ? w0 : d.w[sl]);
    }
    __syncthreads();
    for (int r = r0; r < nrows; r += NT) {
        float acc = ordered_sum_from(part[r * NCB], part + r * NCB, d.R * NCB, d.n_slots);
        const size_t q = row0 + r;
        if (d.shared) acc = __fadd_rn(acc, r == r0 ? sh0 : d.shared[q]);
        if (d.resid) acc = __fadd_rn(r == r0 ? rs0 : d.resid[q], acc);
        if (d.accumulate) acc = __fadd_rn(r == r0 ? ac0 : o[r], acc);
        o[r] = acc;
    }
}

template <int NT>
__global__ __launch_bounds__(NT) void k_layer_decode(LayerArgs a) {
    constexpr int QT = QT_IQ3_S;
    SABAH_STATIC_LDS(QT)
    extern __shared__ __align__(16) uint8_t smem[];
    const int b = (int)blockIdx.x;
    if (b < a.n_g) {
        // ---- gate/up + SwiGLU: rows of one slot, published for the down workgroups
        __builtin_amdgcn_s_setprio(1);                      // ahead of the down waves on a shared SIMD
        const uint32_t target = a.sync[b] + 1u;
        const int tile = b % a.g_tiles, s = b / a.g_tiles;
        gate_up_rounds_tile<QT, NT, 2>(a.gu, 0, s, tile * a.gu.R, tabs, smem, stage, true);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");    // this thread's h stores are in memory
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(a.sync + b, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ---- down + routed combine of rows row0 .. row0 + R (k_down_combine's steps)
    const DownArgs& d = a.dn;
    const int dj = b - a.n_g;
    uint32_t* my = a.sync + kSyncDOff + dj;
    const uint32_t target = *my + 1u;
    // this workgroup's XCD, and its leader ticket taken at once (the returned
    // value is first needed at the wait, after the weights are staged)
    const unsigned x = a.xcd_groups ? (unsigned)(dj % a.xcd_groups) : xcc_id();
    uint32_t ticket = target;
    if (threadIdx.x == 0)
        ticket = __hip_atomic_exchange(a.sync + kSyncT + kLine * x, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (dj == 0) {                                          // advance the entries no workgroup of this launch owns
        for (int i = a.n_g + (int)threadIdx.x; i < kSyncG; i += NT) a.sync[i] = target;
        for (int i = a.n_d + (int)threadIdx.x; i < kSyncD; i += NT) a.sync[kSyncDOff + i] = target;
    }
    const int NCB = contribs_per_row(QT, d.d_ff);
    const Plan P = make_plan(QT, d.d_ff, d.n_slots, d.n_slots * d.R * NCB);
    const int row0 = dj * d.R;
    const int nrows = min(d.R, d.d_model - row0);
    const size_t rb = row_bytes(QT, d.d_ff);
    uint8_t* act = smem + P.off_act;
    float* part = reinterpret_cast<float*>(smem + P.off_part);
    // lane s of every wave holds slot s's tile (lanes past n_slots repeat the
    // last slot); a slot with an invalid id stages expert 0's rows, never used
    const int lane = (int)(threadIdx.x & 63u);
    const SlotWord sw = load_slot_word(d.D, d.rt, 0, min(lane, d.n_slots - 1), d.n_slots);
    __builtin_amdgcn_sched_barrier(0);
    const float* wt = d.w;
    const float rcp_r = __builtin_amdgcn_rcpf((float)d.R);
    const int i0 = (int)threadIdx.x, r0 = (int)threadIdx.x;
    const float w0 = i0 < d.n_slots * d.R ? wt[div_small(i0, rcp_r)] : 0.0f;
    const size_t orow = (size_t)row0 + r0;
    const float sh0 = d.shared && r0 < nrows ? d.shared[orow] : 0.0f;
    const float rs0 = d.resid && r0 < nrows ? d.resid[orow] : 0.0f;
    const float ac0 = d.accumulate && r0 < nrows ? d.out[orow] : 0.0f;
    // wait d_delay, then the codebook table: this workgroup's weight loads
    // then queue behind the gate/up workgroups', whose bytes are needed sooner
    if (a.d_delay) {
        const unsigned long long t0 = wall_ticks();
        while (wall_ticks() - t0 < a.d_delay) __builtin_amdgcn_s_sleep(8);
    }
    store_tables<QT, NT>(tabs, load_tables<QT, NT>((int)threadIdx.x), (int)threadIdx.x);
    const uint8_t* e = resolve_slot_word(d.D, d.rt, sw);
    const bool bad = __any(e == nullptr);
    const uint8_t* mine = (e ? e : d.D.base) + (size_t)row0 * rb;
    auto tile_ptr = [&](int m) { return lane_ptr(mine, m); };
    TileRun<QT, NT> S{TileWalk<QT, NT>(d.n_slots, nrows, rb, d.d_ff)};
    tiles_begin(S, tile_ptr);                               // the whole tile in one pass (checked by the host)
    pass_store(S, stage, leads);
    __syncthreads();                                        // staged units and table written
    // While gate/up runs: each lane pair's unit (tile-major, as pass_decode
    // numbers them; at most one per pair, checked by the host) decoded to
    // int8 weights in registers, half a unit per lane.
    const int u = (int)threadIdx.x >> 1, half = (int)threadIdx.x & 1;
    const bool has = u < S.T.n_mat * S.nv;                  // alike for both lanes of a pair
    Iq3sHalf W;
    uint32_t dbits = 0;
    int ut = 0, ur = 0, us = 0;
    if (has) {
        ut = div_small(u, __builtin_amdgcn_rcpf((float)S.nv));
        const int v = S.v0 + (u - ut * S.nv);
        ur = div_small(v, S.T.rcp_nus);
        us = v - ur * S.T.NUS;
        const uint8_t* unit = stage + 16 * S.cpt * ut + leads[ut] + (int)((size_t)ur * S.T.rb) +
                              us * UnitFmt<QT>::BYTES - S.b0;
        uint32_t G[UnitFmt<QT>::NF];
        iq3s_half_fields(unit, half, G, dbits);
        iq3s_half_decode(G, tabs, W);
    }
    __shared__ int ok;
    if (threadIdx.x < 64) {
        const bool done = layer_wait_h(a, target, x, ticket);
        if (threadIdx.x == 0) ok = done ? 1 : 0;
    }
    __syncthreads();                                        // flags seen
    float* o = d.out + row0;
    if (!ok) {
        if (threadIdx.x == 0) *reinterpret_cast<volatile unsigned int*>(d.err) = kErrLayerWait;
        for (int r = threadIdx.x; r < nrows; r += NT) o[r] = __builtin_nanf("");
        if (threadIdx.x == 0) *my = target;
        return;
    }
    const ActBatch hb{d.h, (size_t)d.d_ff, d.n_slots, d.d_ff, act_type(QT), act, P.act_bytes};
    ActRegs<1> ha;
    act_prefetch<1, NT>(hb, ha);
    act_quantize<1, NT>(hb, ha);
    __syncthreads();                                        // q8 h rows ready
    if (has) {
        const uint8_t* arow = act + ut * P.act_bytes;
        uint32_t A[4][8];
        act_half(arow + us * kActChunkStride, half, A);
        int bs = iq3s_half_dot(W, A);
        bs += (int)dpp<kDppXor1>((uint32_t)bs);             // the partner lane's half
        if (half == 0) {
            const ActLayout AL(d.d_ff, QT_Q8_K);
            part[(ut * d.R + ur) * NCB + us] =
                __fmul_rn(__fmul_rn(h2f(dbits), reinterpret_cast<const float*>(arow + AL.off_d)[us]), (float)bs);
        }
    }
    __syncthreads();
    if (bad) {
        flag_error(d.err);
        for (int r = threadIdx.x; r < nrows; r += NT) o[r] = __builtin_nanf("");
        if (threadIdx.x == 0) *my = target;
        return;
    }
    layer_combine(d, NCB, nrows, part, o, (size_t)row0, w0, sh0, rs0, ac0, NT);
    if (threadIdx.x == 0) *my = target;
}

// every entry of the lockstep flags to zero (at init, and after a wait ran out)
__global__ void k_clear_sync(uint32_t* sync) {
    for (int i = threadIdx.x; i < kSyncWords; i += blockDim.x) sync[i] = 0u;
}

}  // namespace sabah
