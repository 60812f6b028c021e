// sabah_rt: C-ABI entry points of the MI355X expert runtime (include/sabah_rt.h).
//
// Host side of the hooked operator.  Compared with the reference runtime
// (sabah_rt.cu:3494-3833) the per-call host work is reduced to argument
// validation, one address lookup and one kernel launch: the bank is resident
// in HBM, the ids are read by the kernel itself, and there is no pointer
// table upload, copy stream or stream drain.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_set>
#include <vector>

#include "dense_kernels.h"
#include "host_decode.h"
#include "layer_kernels.h"
#include "mmid_kernels.h"
#include "prefill_kernels.h"
#include "route_kernels.h"
#include "synth_kernels.h"
#include "sabah_rt.h"

#define SABAH_API extern "C" __attribute__((visibility("default")))

using namespace sabah;

// The library's static device array, one per GPU: the fused decode layer's
// lockstep flags (k_layer_decode; persistent, cleared at init), then the
// 8 MiB arena of sabah_moe_layer_noalloc's per-call scratch.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
constexpr size_t kSyncBytes = (size_t)kSyncWords * 4;
static_assert(kSyncBytes % 256 == 0, "the arena after the flags stays 256-byte aligned");
static __device__ __align__(256) uint8_t scratch[kSyncBytes + kNoAllocScratchBytes];

namespace {

char g_err[512] = {0};
std::mutex g_mu;
int g_device = -1;
hipStream_t g_stream = nullptr;
hipStream_t g_copy = nullptr;     // the harness's copy stream (sabah_h2d_async, sabah_event_record_copy)
// A batch layer's shared expert runs on g_side, forked from the caller's
// stream at the layer's start (g_ev_fork) and joined before the launch that
// adds its output (g_ev_join), so it overlaps the routed gate/up.  The fork,
// the shared launches and the join's wait are issued under g_side_mu, so
// layers issued from several threads do not interleave their event records.
hipStream_t g_side = nullptr;
hipEvent_t g_ev_fork = nullptr, g_ev_join = nullptr;
std::mutex g_side_mu;
unsigned int* g_err_host = nullptr;   // host-mapped sticky error word
unsigned int* g_err_dev = nullptr;    // its device address

struct BankEntry {
    uintptr_t key;
    size_t bytes;
    uint8_t* dev;
    size_t expert_stride;
    int n_experts;
};
std::vector<BankEntry> g_banks;
std::unordered_set<uintptr_t> g_device_sources;   // sources already proven to be device memory

std::atomic<unsigned long long> g_calls{0}, g_empty_calls{0}, g_tokens{0}, g_lookups{0}, g_layer_calls{0};

// Sampled self-check of sabah_rt_mul_mat_id_v2 (the reference's
// sb_selfcheck, sabah_rt.cu:3435-3492): after each call, k (token, slot)
// outputs are recomputed on the host in float64 from the expert's bytes and
// the call's input row, quantised as the kernels quantise it (host_decode.h),
// and compared by relative L2 error.  Enabled by SABAH_LLAMA_SELFCHECK=k (or
// SABAH_RT_SELFCHECK) with SABAH_LLAMA_SELFCHECK_TOL, or sabah_rt_set_selfcheck.
// g_sc_sentinel (tests only) perturbs the host recomputation's mapping: 1 the
// neighbouring expert, 2 the next slot's input row, 3 the next token's input
// row; a check that catches those catches a kernel that makes them.
std::atomic<int> g_sc_k{0}, g_sc_sentinel{0};
double g_sc_tol = 1e-5;
std::atomic<unsigned long long> g_sc_ok{0}, g_sc_fail{0}, g_sc_calls{0};
double g_sc_max = 0.0;                           // guarded by g_sc_mu
std::mutex g_sc_mu;
// MUL_MAT_ID calls that took the grouped (expert-major) path
std::atomic<unsigned long long> g_grouped_calls{0};

// grow-only device scratch, one per purpose
struct Scratch {
    void* p = nullptr;
    size_t bytes = 0;
};
Scratch g_scratch_h, g_scratch_hs, g_scratch_ys, g_scratch_hq;
// the shared expert over several tokens: x and h quantised once, the gate logits
Scratch g_scratch_sxq, g_scratch_shq, g_scratch_sgl;
// grouped (prefill) layer: offsets, pair maps, q8 rows of x and h, h and y in group order
Scratch g_scratch_goff, g_scratch_gpair, g_scratch_gxq, g_scratch_gh, g_scratch_ghq, g_scratch_gy;
uint16_t* g_nearest_dev = nullptr;   // IQ3_S encoder table, uploaded on first use

// Optional HIP-event timing of every kernel the library launches, by kernel
// kind (the reference's SABAH_LLAMA_EVENTS probe, sabah_rt.cu:118-151): each
// dispatch records its own start/stop event pair (launch_kernel); elapsed
// times are collected when the caller asks for them.
enum KernelKind { KK_MMID = 0, KK_GATE_UP = 1, KK_DOWN = 2, KK_CHAIN = 3, KK_GGATE_UP = 4, KK_GDOWN = 5, KK_LAYER = 6,
                  KK_COUNT = 7 };
struct EvPair {
    hipEvent_t a, b;
    int kind;
};
std::atomic<bool> g_timing{false};
// set by the calling thread during sabah_moe_layer_noalloc: its launches create no timing events
thread_local bool g_launch_plain = false;
// the timing events' pools (launches from several threads)
std::mutex g_ev_mu;
std::vector<EvPair> g_ev_free, g_ev_pending;
double g_kind_ms[KK_COUNT] = {0};
unsigned long long g_kind_launches[KK_COUNT] = {0};

// Launch a kernel; with kernel timing on, the dispatch itself records a
// start and a stop event (hipExtLaunchKernelGGL), so the pair brackets that
// kernel's execution on its stream and nothing else.
template <typename K, typename... A>
void launch_kernel(int kind, K kernel, dim3 grid, dim3 block, int lds, hipStream_t st, A... args) {
    if (g_timing.load() && !g_launch_plain) {
        std::lock_guard<std::mutex> lk(g_ev_mu);
        if (g_ev_free.empty()) {
            EvPair p{};
            if (hipEventCreate(&p.a) == hipSuccess && hipEventCreate(&p.b) == hipSuccess) g_ev_free.push_back(p);
        }
        if (!g_ev_free.empty()) {
            EvPair ev = g_ev_free.back();
            g_ev_free.pop_back();
            ev.kind = kind;
            hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, ev.a, ev.b, 0u, args...);
            g_ev_pending.push_back(ev);
            return;
        }
    }
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

bool ck(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
    return false;
}

// a stream argument is used as given: NULL is the HIP null stream, as in any
// HIP API (the entry points without a stream argument use the library stream)
hipStream_t pick_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Scratch that has been outgrown is retired, not freed: a HIP graph captured
// earlier still holds its address and reads it on every replay, so it lives
// until sabah_rt_shutdown.  Growth allocates, which a stream capture cannot
// record: during a capture a call that needs more scratch than any call
// before it fails and names the size (make the same call once outside the
// capture first).
std::vector<void*> g_retired;
size_t g_scratch_total = 0;   // bytes of every grow-only buffer allocated (live and retired)

bool stream_capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return cs != hipStreamCaptureStatusNone;
}

void* grow_scratch(Scratch& s, size_t bytes, hipStream_t stream) {
    if (s.bytes >= bytes) return s.p;
    if (stream_capturing(stream)) {
        fail("library scratch must grow to %zu bytes (from %zu) during a stream capture, which cannot "
             "allocate: make the same call once before the capture", bytes, s.bytes);
        return nullptr;
    }
    size_t want = std::max(bytes, std::max(2 * s.bytes, (size_t)1 << 20));
    void* p = nullptr;
    if (!ck(hipMalloc(&p, want), "scratch allocation")) return nullptr;
    if (s.p) g_retired.push_back(s.p);
    s.p = p;
    s.bytes = want;
    g_scratch_total += want;
    return s.p;
}

// The fixed device array `scratch`, which each GPU the library runs on holds
// until the process ends: its flags (g_layer_sync) and its arena
// (g_noalloc_scratch, sabah_moe_layer_noalloc's scratch).  In host code the
// array's name is a host-side stand-in, not a device address: host code uses
// only the address hipGetSymbolAddress gives at sabah_rt_init, kept per device.
constexpr int kMaxDevices = 64;
void* g_noalloc_scratch[kMaxDevices] = {};
uint32_t* g_layer_sync[kMaxDevices] = {};
// 1 (default): one-token IQ3_S layers run as one fused launch
// (k_layer_decode) when eligible; 0: always the two-kernel form.  The
// results are bit-identical; on the 48-layer decode the fused launch
// measured 1,510 GB/s against 1,433 - 1,449 (same box, interleaved runs).
std::atomic<int> g_layer_fusion{1};
// 1 (default): IQ3_S MUL_MAT_ID calls whose row tiles stay single-pass (one
// token, or a few) run k_mmid_rounds; 0: k_mmid.  The results are bit-identical.
std::atomic<int> g_mmid_rounds{1};
// set when a fused launch's wait ran out: the next fused launch first clears the flags
std::atomic<bool> g_sync_reset_pending{false};
// one-shot test of the timeout path (sabah_rt_set_layer_fusion(2))
std::atomic<bool> g_layer_wait_test{false};
// placement test of the fused layer (sabah_rt_set_layer_placement_test): 0, or
// g > 0 to group down workgroup j with XCD j % g instead of its hardware XCD
std::atomic<int> g_layer_xcd_groups{0};

// LDS a workgroup may allocate (the device's limit: 160 KB on gfx950)
int g_max_lds = 65536;
// compute units of the device (256 on MI355X)
int g_num_cu = 256;

// Launches above 64 KB of LDS (static + dynamic) declare their dynamic size to
// the runtime first.
template <typename K>
hipError_t fit_lds(K kernel, int bytes, int total) {
    if (total > g_max_lds) return hipErrorInvalidConfiguration;
    if (total > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// rows per workgroup (rows_per_wg); rows that are not packed are one tile
// each, at most kMaxTiles per workgroup
int rows_mmid(int qt, int k, bool packed) {
    return packed ? rows_per_wg(qt, k, 1) : std::min(kMaxTiles, rows_per_wg(qt, k, 1));
}
// Rows per workgroup of the tile kernels: the tile one pass stages (r0), or a
// multiple of it while the launch keeps at least kMinWorkgroups workgroups:
// with several tokens per launch there are workgroups to spare, and a
// workgroup that walks its tiles in several passes (the next pass loading
// while the current one decodes) spreads its fixed costs (expert ids, q8
// activations, codebook table, epilogue) over more rows.  Measured on the
// mixed 32-token layer (Q4_K gate/up, Q6_K down): gate/up 75 -> 62 us at 8
// passes (16 passes: 67 us), down 213 -> 135 us at 13 passes (8: 149 us).
constexpr int kMinWorkgroups = 1024;
constexpr int kMaxPassesGateUp = 8, kMaxPassesDown = 16;
// lds_of(R): the launch's LDS at R rows per workgroup (the partials grow with R)
template <typename F>
int grow_rows(int r0, int rows, long long wg_per_row_tile, int max_passes, F lds_of) {
    int m = 1;
    while (m < max_passes && r0 * (m + 1) <= rows &&
           (long long)((rows + r0 * (m + 1) - 1) / (r0 * (m + 1))) * wg_per_row_tile >= kMinWorkgroups &&
           lds_of(r0 * (m + 1)) <= g_max_lds)
        ++m;
    return r0 * m;
}
// One token: the row tile r0 shrunk (to no less than half) while that raises
// the launch's workgroups to the next multiple of the CU count, so every CU
// gets the same share: a launch of 384 workgroups leaves half the CUs with
// two, one of 128 leaves half of them idle.  Measured on the one-token
// layers (48 calls in a replayed graph): Q8_0 E=8 top-2 (down 128 -> 256
// workgroups) 10.97 against 11.18 us, Q4_K E=128 top-8 (gate/up 384 -> 512,
// down 205 -> 256) 12.31 against 12.76 us per layer.
int balance_rows(int r0, int rows, long long groups) {
    const long long wg = (rows + r0 - 1) / r0 * groups;
    const long long target = (wg + g_num_cu - 1) / g_num_cu * g_num_cu;
    for (int r = r0; 2 * r >= r0; --r)
        if ((rows + r - 1) / r * groups >= target) return r;
    return r0;
}
int rows_gate_up(int qt, int k, int d_ff, int n_slots, int n_tokens) {
    if (gate_up_rounds_ok(qt, k)) return rows_gate_up_rounds(qt, k);
    if (n_tokens == 1) return balance_rows(rows_per_wg(qt, k, 2), d_ff, n_slots);
    return grow_rows(rows_per_wg(qt, k, 2), d_ff, (long long)n_slots * n_tokens, kMaxPassesGateUp,
                     [&](int r) { return launch_lds(qt, make_plan(qt, k, 1, 2 * r * contribs_per_row(qt, k))); });
}
int rows_down(int qt, int k, int n_slots, int d_model, int n_tokens) {
    if (n_tokens == 1) return balance_rows(rows_per_wg(qt, k, n_slots), d_model, 1);
    return grow_rows(rows_per_wg(qt, k, n_slots), d_model, n_tokens, kMaxPassesDown, [&](int r) {
        return launch_lds(qt, make_plan(qt, k, n_slots, n_slots * r * contribs_per_row(qt, k)));
    });
}

bool check_sticky() {
    const unsigned int w = g_err_host ? __atomic_load_n(g_err_host, __ATOMIC_ACQUIRE) : 0u;
    if (w == 0) return true;
    __atomic_store_n(g_err_host, 0u, __ATOMIC_RELEASE);
    if (w == kErrLayerWait) {
        g_sync_reset_pending = true;
        fail("an earlier fused layer kernel's down workgroups waited too long for its gate/up workgroups "
             "(calls overlapping on different streams?); their rows were set to NaN");
    } else {
        fail("an earlier expert kernel read an expert id outside [0, n_experts); "
             "its slot outputs were set to NaN");
    }
    return false;
}

// Resolve a MUL_MAT_ID source to device memory: a registered bank range, or a
// device pointer (checked once per distinct address).
const uint8_t* resolve_source(const void* source, size_t need_bytes) {
    const uintptr_t s = reinterpret_cast<uintptr_t>(source);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (const BankEntry& b : g_banks) {
            if (s >= b.key && s < b.key + b.bytes) {
                if (s - b.key + need_bytes > b.bytes) {
                    fail("expert tensor %p extends past its registered bank (%zu bytes)", source, b.bytes);
                    return nullptr;
                }
                return b.dev + (s - b.key);
            }
        }
        if (g_device_sources.count(s)) return reinterpret_cast<const uint8_t*>(source);
    }
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, source);
    if (e != hipSuccess) (void)hipGetLastError();
    if (e == hipSuccess && attr.type == hipMemoryTypeDevice) {
        std::lock_guard<std::mutex> lk(g_mu);
        g_device_sources.insert(s);
        return reinterpret_cast<const uint8_t*>(source);
    }
    fail("expert tensor %p is neither a registered bank nor device memory "
         "(register it with sabah_rt_register_bank)", source);
    return nullptr;
}

bool sync_ids_enabled() {
    static const int on = [] {
        const char* v = std::getenv("SABAH_RT_SYNC_IDS");
        return (v && *v && *v != '0') ? 1 : 0;
    }();
    return on != 0;
}

template <int QT>
hipError_t launch_mmid(const MmidArgs& a, hipStream_t st) {
    if constexpr (QT == QT_IQ3_S) {
        // a decode step's gate, up or down node, or a few tokens' (the row tiles single-pass,
        // not grown): per-wave rounds
        if (a.R == rows_mmid_rounds(QT, a.k) && g_mmid_rounds.load() &&
            mmid_rounds_ok(QT, a.k, a.row_stride, a.sg_w != nullptr)) {
            constexpr int NT = kMmidRoundThreads;
            const Plan P = make_plan(QT, a.k, 1, a.R * contribs_per_row(QT, a.k));
            if (const hipError_t e = fit_lds(k_mmid_rounds<NT>, P.bytes, kMmidRoundStaticLds + P.bytes))
                return e;
            dim3 grid((unsigned)((a.rows + a.R - 1) / a.R), (unsigned)a.n_ids, (unsigned)a.n_tokens);
            launch_kernel(KK_MMID, k_mmid_rounds<NT>, grid, dim3(NT), P.bytes, st, a);
            return hipGetLastError();
        }
    }
    const Plan P = make_plan(QT, a.k, 1, a.R * contribs_per_row(QT, a.k));
    if (const hipError_t e = fit_lds(k_mmid<QT>, P.bytes, launch_lds(QT, P))) return e;
    dim3 grid((unsigned)((a.rows + a.R - 1) / a.R), (unsigned)a.n_ids, (unsigned)a.n_tokens);
    launch_kernel(KK_MMID, k_mmid<QT>, grid, dim3(kThreads), P.bytes, st, a);
    return hipGetLastError();
}

hipError_t dispatch_mmid(int qt, const MmidArgs& a, hipStream_t st) {
    switch (qt) {
    case QT_Q8_0: return launch_mmid<QT_Q8_0>(a, st);
    case QT_Q4_K: return launch_mmid<QT_Q4_K>(a, st);
    case QT_Q5_K: return launch_mmid<QT_Q5_K>(a, st);
    case QT_Q5_1: return launch_mmid<QT_Q5_1>(a, st);
    case QT_Q6_K: return launch_mmid<QT_Q6_K>(a, st);
    case QT_IQ3_S: return launch_mmid<QT_IQ3_S>(a, st);
    case QT_IQ3_XXS: return launch_mmid<QT_IQ3_XXS>(a, st);
    case QT_IQ4_NL: return launch_mmid<QT_IQ4_NL>(a, st);
    case QT_Q2_0: return launch_mmid<QT_Q2_0>(a, st);
    case QT_IQ4_XS: return launch_mmid<QT_IQ4_XS>(a, st);
    case QT_IQ2_S: return launch_mmid<QT_IQ2_S>(a, st);
    }
    return hipErrorInvalidValue;
}

template <int QT>
hipError_t launch_gate_up(const GateUpArgs& a, int n_tokens, hipStream_t st) {
    const Plan P = make_plan(QT, a.d_model, 1, 2 * a.R * contribs_per_row(QT, a.d_model));
    dim3 grid((unsigned)((a.d_ff + a.R - 1) / a.R), (unsigned)a.n_slots, (unsigned)n_tokens);
    if constexpr (QT == QT_IQ3_S) {
        if (gate_up_rounds_ok(QT, a.d_model) && a.R == rows_gate_up_rounds(QT, a.d_model)) {
            constexpr int NT = kGateUpRoundThreads;
            const int dyn = gate_up_rounds_lds(P, GateUpRounds<QT, NT, 2>::STAGE);
            if (const hipError_t e = fit_lds(k_gate_up_rounds<QT, NT>, dyn, kLdsTables + dyn)) return e;
            launch_kernel(KK_GATE_UP, k_gate_up_rounds<QT, NT>, grid, dim3(NT), dyn, st, a);
            return hipGetLastError();
        }
    }
    if constexpr (QT == QT_Q4_K) {
        // one token: two lanes per unit in 512-thread workgroups (pass_decode; 116 against 191
        // VGPRs).  Measured on the Q4_K E=128 top-8 layer: 12.17 against 12.32 us; with many
        // tokens (grown row tiles, 8 passes) the 256-thread form is faster (32-token mixed
        // layer: routed gate/up 10 % slower split).
        if (n_tokens == 1) {
            constexpr int NT = 2 * kThreads;
            if (const hipError_t e = fit_lds(k_gate_up<QT, NT>, P.bytes, launch_lds(QT, P))) return e;
            launch_kernel(KK_GATE_UP, k_gate_up<QT, NT>, grid, dim3(NT), P.bytes, st, a);
            return hipGetLastError();
        }
    }
    if (const hipError_t e = fit_lds(k_gate_up<QT>, P.bytes, launch_lds(QT, P))) return e;
    launch_kernel(KK_GATE_UP, k_gate_up<QT>, grid, dim3(kThreads), P.bytes, st, a);
    return hipGetLastError();
}

hipError_t dispatch_gate_up(int qt, const GateUpArgs& a, int n_tokens, hipStream_t st) {
    switch (qt) {
    case QT_Q8_0: return launch_gate_up<QT_Q8_0>(a, n_tokens, st);
    case QT_Q4_K: return launch_gate_up<QT_Q4_K>(a, n_tokens, st);
    case QT_Q5_K: return launch_gate_up<QT_Q5_K>(a, n_tokens, st);
    case QT_Q5_1: return launch_gate_up<QT_Q5_1>(a, n_tokens, st);
    case QT_Q6_K: return launch_gate_up<QT_Q6_K>(a, n_tokens, st);
    case QT_IQ3_S: return launch_gate_up<QT_IQ3_S>(a, n_tokens, st);
    case QT_IQ3_XXS: return launch_gate_up<QT_IQ3_XXS>(a, n_tokens, st);
    case QT_IQ4_NL: return launch_gate_up<QT_IQ4_NL>(a, n_tokens, st);
    case QT_Q2_0: return launch_gate_up<QT_Q2_0>(a, n_tokens, st);
    case QT_IQ4_XS: return launch_gate_up<QT_IQ4_XS>(a, n_tokens, st);
    case QT_IQ2_S: return launch_gate_up<QT_IQ2_S>(a, n_tokens, st);
    }
    return hipErrorInvalidValue;
}

template <int QT>
hipError_t launch_down(const DownArgs& a, int n_tokens, hipStream_t st) {
    // IQ3_S runs 512 threads, two lanes per unit (twice the waves to hide the decode's LDS latency)
    constexpr int NT = QT == QT_IQ3_S ? 2 * kThreads : kThreads;
    const Plan P = make_plan(QT, a.d_ff, a.n_slots, a.n_slots * a.R * contribs_per_row(QT, a.d_ff));
    dim3 grid((unsigned)((a.d_model + a.R - 1) / a.R), (unsigned)n_tokens);
    if constexpr (QT == QT_Q4_K) {
        if (n_tokens == 1 && !a.hq) {                       // one token: two lanes per unit, as for gate/up
            if (const hipError_t e = fit_lds(k_down_combine<QT, 2 * kThreads>, P.bytes, launch_lds(QT, P))) return e;
            launch_kernel(KK_DOWN, k_down_combine<QT, 2 * kThreads>, grid, dim3(2 * kThreads), P.bytes, st, a);
            return hipGetLastError();
        }
    }
    if (a.hq) {
        if (const hipError_t e = fit_lds(k_down_combine<QT, NT, true>, P.bytes, launch_lds(QT, P))) return e;
        launch_kernel(KK_DOWN, k_down_combine<QT, NT, true>, grid, dim3(NT), P.bytes, st, a);
        return hipGetLastError();
    }
    if (const hipError_t e = fit_lds(k_down_combine<QT, NT>, P.bytes, launch_lds(QT, P))) return e;
    launch_kernel(KK_DOWN, k_down_combine<QT, NT>, grid, dim3(NT), P.bytes, st, a);
    return hipGetLastError();
}

hipError_t dispatch_down(int qt, const DownArgs& a, int n_tokens, hipStream_t st) {
    switch (qt) {
    case QT_Q8_0: return launch_down<QT_Q8_0>(a, n_tokens, st);
    case QT_Q4_K: return launch_down<QT_Q4_K>(a, n_tokens, st);
    case QT_Q5_K: return launch_down<QT_Q5_K>(a, n_tokens, st);
    case QT_Q5_1: return launch_down<QT_Q5_1>(a, n_tokens, st);
    case QT_Q6_K: return launch_down<QT_Q6_K>(a, n_tokens, st);
    case QT_IQ3_S: return launch_down<QT_IQ3_S>(a, n_tokens, st);
    case QT_IQ3_XXS: return launch_down<QT_IQ3_XXS>(a, n_tokens, st);
    case QT_IQ4_NL: return launch_down<QT_IQ4_NL>(a, n_tokens, st);
    case QT_Q2_0: return launch_down<QT_Q2_0>(a, n_tokens, st);
    case QT_IQ4_XS: return launch_down<QT_IQ4_XS>(a, n_tokens, st);
    case QT_IQ2_S: return launch_down<QT_IQ2_S>(a, n_tokens, st);
    }
    return hipErrorInvalidValue;
}

int validate_mmid(const void* source, const void* d_x, const void* d_ids, const float* d_dst, int x_rows,
                  int n_ids, int n_tokens, int rows, int k, int n_experts, int qt, size_t row_stride) {
    if (!source || !d_x || !d_ids || !d_dst) return fail("invalid Sabah MUL_MAT_ID arguments (null pointer)");
    if (n_tokens < 0 || k <= 0 || rows <= 0 || n_ids <= 0 || n_experts <= 0 || (k % 32) != 0)
        return fail("invalid Sabah MUL_MAT_ID geometry (k=%d rows=%d n_ids=%d n_tokens=%d n_experts=%d)",
                    k, rows, n_ids, n_tokens, n_experts);
    if (x_rows <= 0 || (x_rows != 1 && x_rows != n_ids))
        return fail("Sabah MUL_MAT_ID input rows %d must be 1 (broadcast) or n_ids %d", x_rows, n_ids);
    if (!supported_weight_type(qt)) return fail("unsupported quant type %d (supported: 8 Q8_0, 12 Q4_K, 14 Q6_K, 18 IQ3_XXS, 20 IQ4_NL, 21 IQ3_S, "
                                            "22 IQ2_S, 23 IQ4_XS, 42 Q2_0)", qt);
    if (k % block_elems(qt)) return fail("k=%d is not a whole number of type-%d blocks", k, qt);
    if (row_stride < row_bytes(qt, k)) return fail("row stride %zu is shorter than a row (%zu bytes)", row_stride, row_bytes(qt, k));
    return 0;
}

// ---------------------------------------------------------------------------
// Device slab: one allocation carved into ranges (the reference's slab,
// sabah_rt.cu:332-420, serves its VRAM tier; here it serves harness callers
// that bind it).  Free ranges are kept by offset and merged with their
// neighbours on free; allocation takes the smallest free range that fits.
// ---------------------------------------------------------------------------
std::mutex g_slab_mu;
uint8_t* g_slab = nullptr;
size_t g_slab_cap = 0;
std::map<size_t, size_t> g_slab_free_ranges;     // offset -> bytes
std::map<size_t, size_t> g_slab_used;            // offset -> bytes
constexpr size_t kSlabAlign = 256;

void slab_release() {
    std::lock_guard<std::mutex> lk(g_slab_mu);
    if (g_slab) (void)hipFree(g_slab);
    g_slab = nullptr;
    g_slab_cap = 0;
    g_slab_free_ranges.clear();
    g_slab_used.clear();
}

}  // namespace

// ===========================================================================
// lifecycle
// ===========================================================================
SABAH_API const char* sabah_rt_last_error(void) { return g_err; }

SABAH_API const char* sabah_rt_build_info(void) { return "sabah_rt abi=v2 sentinel=0 arch=gfx950"; }

SABAH_API int sabah_rt_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

static void report_trace_at_exit();

SABAH_API int sabah_rt_init(int device) {
    if (g_device == device && g_stream) return 0;
    if (g_device >= 0) return fail("sabah_rt_init(%d): already initialised on device %d", device, g_device);
    if (!ck(hipSetDevice(device), "hipSetDevice")) return -1;
    int lds = 0;
    if (!ck(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device), "LDS limit")) return -1;
    g_max_lds = lds;
    int cus = 0;
    if (!ck(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device), "CU count")) return -1;
    g_num_cu = std::max(1, cus);
    if (!ck(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "create stream")) return -1;
    if (!ck(hipStreamCreateWithFlags(&g_copy, hipStreamNonBlocking), "create copy stream")) return -1;
    if (!ck(hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking), "create shared-expert stream") ||
        !ck(hipEventCreateWithFlags(&g_ev_fork, hipEventDisableTiming), "create fork event") ||
        !ck(hipEventCreateWithFlags(&g_ev_join, hipEventDisableTiming), "create join event"))
        return -1;
    if (!ck(hipHostMalloc(reinterpret_cast<void**>(&g_err_host), sizeof(unsigned int), hipHostMallocMapped),
            "sticky error word")) return -1;
    *g_err_host = 0;
    if (!ck(hipHostGetDevicePointer(reinterpret_cast<void**>(&g_err_dev), g_err_host, 0), "sticky error word map"))
        return -1;
    if (device >= 0 && device < kMaxDevices && !g_noalloc_scratch[device]) {
        static_assert(sizeof(scratch) == kSyncBytes + kNoAllocScratchBytes, "the static array has its stated size");
        void* p = nullptr;
        if (!ck(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch address")) return -1;
        uint32_t* flags = static_cast<uint32_t*>(p);
        hipLaunchKernelGGL(k_clear_sync, dim3(1), dim3(256), 0, g_stream, flags);
        if (!ck(hipGetLastError(), "layer flags clear") || !ck(hipStreamSynchronize(g_stream), "layer flags clear sync"))
            return -1;
        g_layer_sync[device] = flags;
        g_noalloc_scratch[device] = static_cast<uint8_t*>(p) + kSyncBytes;
    }
    g_device = device;
    {
        const char* k = std::getenv("SABAH_LLAMA_SELFCHECK");
        if (!k || !*k) k = std::getenv("SABAH_RT_SELFCHECK");
        const char* tol = std::getenv("SABAH_LLAMA_SELFCHECK_TOL");
        if (k && *k) g_sc_k.store(std::max(0, std::atoi(k)));
        if (tol && *tol && std::atof(tol) > 0.0) g_sc_tol = std::atof(tol);
        static bool registered = false;
        if (!registered) registered = std::atexit(report_trace_at_exit) == 0;
    }
    return 0;
}

SABAH_API int sabah_rt_shutdown(void) {
    if (g_device < 0) return 0;
    if (g_stream) (void)hipStreamSynchronize(g_stream);
    for (Scratch* s : {&g_scratch_h, &g_scratch_hs, &g_scratch_ys, &g_scratch_hq, &g_scratch_sxq, &g_scratch_shq,
                       &g_scratch_sgl, &g_scratch_goff, &g_scratch_gpair, &g_scratch_gxq, &g_scratch_gh, &g_scratch_ghq,
                       &g_scratch_gy}) {
        if (s->p) (void)hipFree(s->p);
        s->p = nullptr;
        s->bytes = 0;
    }
    for (void* p : g_retired) (void)hipFree(p);
    g_retired.clear();
    g_scratch_total = 0;
    if (g_nearest_dev) (void)hipFree(g_nearest_dev);
    g_nearest_dev = nullptr;
    if (g_err_host) (void)hipHostFree(g_err_host);
    g_err_host = nullptr;
    g_err_dev = nullptr;
    if (g_stream) (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    if (g_copy) (void)hipStreamDestroy(g_copy);
    g_copy = nullptr;
    if (g_side) (void)hipStreamSynchronize(g_side), (void)hipStreamDestroy(g_side);
    g_side = nullptr;
    if (g_ev_fork) (void)hipEventDestroy(g_ev_fork);
    if (g_ev_join) (void)hipEventDestroy(g_ev_join);
    g_ev_fork = g_ev_join = nullptr;
    slab_release();
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_banks.clear();
        g_device_sources.clear();
    }
    g_device = -1;
    return 0;
}

SABAH_API int sabah_sync_all(void) { return ck(hipDeviceSynchronize(), "sync device") ? 0 : -1; }
SABAH_API int sabah_sync_compute(void) {
    if (!g_stream) return fail("sabah_rt_init has not been called");
    return ck(hipStreamSynchronize(g_stream), "sync stream") ? 0 : -1;
}

SABAH_API int sabah_rt_check_errors(void) { return check_sticky() ? 0 : -1; }

SABAH_API int sabah_rt_set_kernel_timing(int on) {
    g_timing = on != 0;
    return 0;
}

// 1 (default): one-token IQ3_S layers run as one fused launch when
// eligible; 0: always gate/up then down + combine.  The results are
// bit-identical.
// 2: as 1, and the next fused launch tests its timeout path: its down
// workgroups wait for a flag value that no workgroup writes, so their
// wait runs out (2 ms without progress), their rows become NaN and the next call
// fails with the message; the flags are then cleared before the next fused
// launch.
SABAH_API int sabah_rt_set_layer_fusion(int mode) {
    if (mode < 0 || mode > 2) return fail("layer fusion mode %d outside {0 off, 1 on, 2 on + timeout test}", mode);
    g_layer_fusion.store(mode == 0 ? 0 : 1);
    g_layer_wait_test.store(mode == 2);
    return 0;
}

// The IQ3_S MUL_MAT_ID kernel of single-pass launches (one token, or a few):
// 1 (default) per-wave rounds (k_mmid_rounds), 0 the whole-tile kernel
// (k_mmid).  The results do not change; tests run both.
SABAH_API int sabah_rt_set_mmid_rounds(int mode) {
    if (mode < 0 || mode > 1) return fail("MUL_MAT_ID rounds mode %d outside {0 off, 1 on}", mode);
    g_mmid_rounds.store(mode);
    return 0;
}

// Placement test of the fused layer: with groups g in 1..8 its down
// workgroups elect one leader per group as if down workgroup j ran on XCD
// j % g (g = 1: all on one XCD; g = 3: five XCDs without any), instead of per
// hardware XCD; 0 restores the hardware grouping.  The results do not change.
SABAH_API int sabah_rt_set_layer_placement_test(int groups) {
    if (groups < 0 || groups > kSyncXcds) return fail("layer placement test groups %d outside [0, %d]", groups, kSyncXcds);
    g_layer_xcd_groups.store(groups);
    return 0;
}

// ===========================================================================
// memory, copies and events for the harness (the reference's rt.py binds
// these by name, rt.py:70-107; semantics as sabah_rt.cu:3240-3353)
// ===========================================================================
SABAH_API void* sabah_dev_alloc(size_t bytes) {
    void* p = nullptr;
    return ck(hipMalloc(&p, bytes), "device allocation") ? p : nullptr;
}
SABAH_API void sabah_dev_free(void* p) {
    if (p) (void)hipFree(p);
}
// pinned host memory (hipHostMalloc), released by sabah_host_free
SABAH_API void* sabah_host_alloc(size_t bytes) {
    void* p = nullptr;
    return ck(hipHostMalloc(&p, bytes, hipHostMallocDefault), "pinned host allocation") ? p : nullptr;
}
SABAH_API void sabah_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}
SABAH_API int sabah_dev_mem(size_t* free_bytes, size_t* total_bytes) {
    return ck(hipMemGetInfo(free_bytes, total_bytes), "device memory info") ? 0 : -1;
}
// The blocking copies and the memset are ordered after everything the
// library's streams hold and complete before they return (the ordering a
// null-stream call has against blocking streams).  The library's streams are
// non-blocking, so a null-stream call alone would not wait for them: each call
// drains the copy stream, then runs on the compute stream and waits for it.
static int ordered_copy(void* dst, const void* src, size_t n, hipMemcpyKind kind, const char* what) {
    if (!g_stream) return ck(hipMemcpy(dst, src, n, kind), what) ? 0 : -1;
    return ck(hipStreamSynchronize(g_copy), what) && ck(hipMemcpyAsync(dst, src, n, kind, g_stream), what) &&
                   ck(hipStreamSynchronize(g_stream), what)
               ? 0
               : -1;
}
SABAH_API int sabah_memcpy_h2d(void* dst, const void* src, size_t n) {
    return ordered_copy(dst, src, n, hipMemcpyHostToDevice, "copy to device");
}
SABAH_API int sabah_memcpy_d2h(void* dst, const void* src, size_t n) {
    return ordered_copy(dst, src, n, hipMemcpyDeviceToHost, "copy to host");
}
SABAH_API int sabah_memset_d(void* dst, int v, size_t n) {
    if (!g_stream) return ck(hipMemset(dst, v, n), "device memset") && ck(hipDeviceSynchronize(), "device memset") ? 0 : -1;
    return ck(hipStreamSynchronize(g_copy), "device memset") && ck(hipMemsetAsync(dst, v, n, g_stream), "device memset") &&
                   ck(hipStreamSynchronize(g_stream), "device memset")
               ? 0
               : -1;
}
// host to device on the library's copy stream (ordered against the compute
// stream only through the event calls below)
SABAH_API int sabah_h2d_async(void* dst, const void* src, size_t n) {
    if (!g_copy) return fail("sabah_rt_init has not been called");
    return ck(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_copy), "async copy to device") ? 0 : -1;
}
SABAH_API void* sabah_event_create(void) {
    hipEvent_t e = nullptr;
    return ck(hipEventCreate(&e), "event create") ? reinterpret_cast<void*>(e) : nullptr;
}
SABAH_API void sabah_event_destroy(void* ev) {
    if (ev) (void)hipEventDestroy(reinterpret_cast<hipEvent_t>(ev));
}
SABAH_API int sabah_event_record_copy(void* ev) {
    if (!g_copy) return fail("sabah_rt_init has not been called");
    return ck(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), g_copy), "record on the copy stream") ? 0 : -1;
}
SABAH_API int sabah_event_record_compute(void* ev) {
    if (!g_stream) return fail("sabah_rt_init has not been called");
    return ck(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), g_stream), "record on the compute stream") ? 0 : -1;
}
SABAH_API int sabah_compute_wait_event(void* ev) {
    if (!g_stream) return fail("sabah_rt_init has not been called");
    return ck(hipStreamWaitEvent(g_stream, reinterpret_cast<hipEvent_t>(ev), 0), "compute stream wait") ? 0 : -1;
}
SABAH_API int sabah_copy_wait_event(void* ev) {
    if (!g_copy) return fail("sabah_rt_init has not been called");
    return ck(hipStreamWaitEvent(g_copy, reinterpret_cast<hipEvent_t>(ev), 0), "copy stream wait") ? 0 : -1;
}
// milliseconds from event a to event b, after b has completed; -1 on error
SABAH_API float sabah_event_elapsed_ms(void* a, void* b) {
    float ms = -1.0f;
    if (!ck(hipEventSynchronize(reinterpret_cast<hipEvent_t>(b)), "event sync")) return -1.0f;
    if (!ck(hipEventElapsedTime(&ms, reinterpret_cast<hipEvent_t>(a), reinterpret_cast<hipEvent_t>(b)),
            "event elapsed time"))
        return -1.0f;
    return ms;
}
SABAH_API int sabah_event_sync(void* ev) {
    return ck(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev)), "event sync") ? 0 : -1;
}
// 1: complete, 0: still in flight, -1: error
SABAH_API int sabah_event_query(void* ev) {
    const hipError_t e = hipEventQuery(reinterpret_cast<hipEvent_t>(ev));
    if (e == hipSuccess) return 1;
    if (e == hipErrorNotReady) {
        (void)hipGetLastError();
        return 0;
    }
    ck(e, "event query");
    return -1;
}
SABAH_API int sabah_sync_copy(void) {
    if (!g_copy) return fail("sabah_rt_init has not been called");
    return ck(hipStreamSynchronize(g_copy), "sync copy stream") ? 0 : -1;
}

// The slab (sabah_rt.cu:3889-3903): one device allocation of capacity_bytes,
// ranges of it handed out 256-byte aligned.  Init on an existing slab is a
// no-op; alloc returns NULL when no free range fits; free of a pointer the
// slab did not hand out does nothing.
SABAH_API int sabah_slab_init(size_t capacity_bytes) {
    std::lock_guard<std::mutex> lk(g_slab_mu);
    if (g_slab) return 0;
    if (capacity_bytes == 0) return fail("slab capacity must be positive");
    void* p = nullptr;
    if (!ck(hipMalloc(&p, capacity_bytes), "slab allocation")) return -1;
    g_slab = static_cast<uint8_t*>(p);
    g_slab_cap = capacity_bytes;
    g_slab_free_ranges = {{0, capacity_bytes}};
    g_slab_used.clear();
    return 0;
}
SABAH_API void* sabah_slab_alloc(size_t bytes) {
    std::lock_guard<std::mutex> lk(g_slab_mu);
    if (!g_slab || bytes == 0) return nullptr;
    const size_t want = (bytes + kSlabAlign - 1) & ~(kSlabAlign - 1);
    auto best = g_slab_free_ranges.end();
    for (auto it = g_slab_free_ranges.begin(); it != g_slab_free_ranges.end(); ++it)
        if (it->second >= want && (best == g_slab_free_ranges.end() || it->second < best->second)) best = it;
    if (best == g_slab_free_ranges.end()) return nullptr;
    const size_t off = best->first, avail = best->second;
    g_slab_free_ranges.erase(best);
    if (avail > want) g_slab_free_ranges[off + want] = avail - want;
    g_slab_used[off] = want;
    return g_slab + off;
}
SABAH_API void sabah_slab_free(void* ptr) {
    std::lock_guard<std::mutex> lk(g_slab_mu);
    if (!g_slab || !ptr) return;
    const uint8_t* p = static_cast<const uint8_t*>(ptr);
    if (p < g_slab || p >= g_slab + g_slab_cap) return;
    auto u = g_slab_used.find((size_t)(p - g_slab));
    if (u == g_slab_used.end()) return;
    size_t off = u->first, len = u->second;
    g_slab_used.erase(u);
    auto next = g_slab_free_ranges.lower_bound(off);
    if (next != g_slab_free_ranges.begin()) {                  // merge with the range before
        auto prev = std::prev(next);
        if (prev->first + prev->second == off) {
            off = prev->first;
            len += prev->second;
            g_slab_free_ranges.erase(prev);
        }
    }
    if (next != g_slab_free_ranges.end() && off + len == next->first) {   // and the one after
        len += next->second;
        g_slab_free_ranges.erase(next);
    }
    g_slab_free_ranges[off] = len;
}
SABAH_API void sabah_slab_destroy(void) { slab_release(); }

// Accumulated kernel time (ms) and launch count of one kernel kind
// (0 MUL_MAT_ID, 1 gate/up, 2 down+combine, 3 decode chain); waits for the
// launches still in flight.  reset != 0 clears the totals after reading.
SABAH_API int sabah_rt_get_kernel_timing(int kind, double* total_ms, unsigned long long* launches, int reset) {
    if (kind < 0 || kind >= KK_COUNT) return fail("unknown kernel kind %d", kind);
    std::lock_guard<std::mutex> lk(g_ev_mu);
    for (EvPair& p : g_ev_pending) {
        float ms = 0.0f;
        if (!ck(hipEventSynchronize(p.b), "timing event sync")) return -1;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            g_kind_ms[p.kind] += ms;
            g_kind_launches[p.kind] += 1;
        }
        g_ev_free.push_back(p);
    }
    g_ev_pending.clear();
    if (total_ms) *total_ms = g_kind_ms[kind];
    if (launches) *launches = g_kind_launches[kind];
    if (reset) {
        for (int i = 0; i < KK_COUNT; ++i) {
            g_kind_ms[i] = 0;
            g_kind_launches[i] = 0;
        }
    }
    return 0;
}

// ===========================================================================
// bank registry
// ===========================================================================
SABAH_API int sabah_rt_register_bank(const void* source_key, void* d_base, size_t bytes, size_t expert_stride,
                                     int n_experts) {
    if (!source_key || !d_base || bytes == 0 || expert_stride == 0 || n_experts <= 0)
        return fail("invalid bank registration");
    if (expert_stride * (size_t)n_experts > bytes)
        return fail("bank of %zu bytes cannot hold %d experts of %zu bytes", bytes, n_experts, expert_stride);
    const uintptr_t k = reinterpret_cast<uintptr_t>(source_key);
    std::lock_guard<std::mutex> lk(g_mu);
    for (const BankEntry& b : g_banks) {
        if (k < b.key + b.bytes && b.key < k + bytes) {
            if (b.key == k && b.bytes == bytes && b.dev == reinterpret_cast<uint8_t*>(d_base)) return 0;
            snprintf(g_err, sizeof(g_err), "bank %p overlaps a registered bank", source_key);
            return -1;
        }
    }
    g_banks.push_back({k, bytes, reinterpret_cast<uint8_t*>(d_base), expert_stride, n_experts});
    return 0;
}

SABAH_API int sabah_rt_unregister_bank(const void* source_key) {
    const uintptr_t k = reinterpret_cast<uintptr_t>(source_key);
    std::lock_guard<std::mutex> lk(g_mu);
    for (size_t i = 0; i < g_banks.size(); ++i) {
        if (g_banks[i].key == k) {
            g_banks.erase(g_banks.begin() + (long)i);
            return 0;
        }
    }
    snprintf(g_err, sizeof(g_err), "bank %p is not registered", source_key);
    return -1;
}

// ===========================================================================
// MUL_MAT_ID
// ===========================================================================
// ---------------------------------------------------------------------------
// Grouped MUL_MAT_ID (IQ3_S, Q4_K, Q6_K, many tokens): the (token, slot) pairs are grouped
// by expert on the device and each expert's rows are read once per call, with
// int8 MFMA over up to 16 pairs at a time.  The integer block sums and every
// fp32 step are the token-major kernel's, so the results are bit-identical to
// it; the choice between the two paths changes no value.
//   mode 0 (default): grouped when eligible and the call has at least
//     grouped_min_pairs(form, qt) pairs per expert on average;
//   mode 1: never; mode 2: whenever eligible.
// ---------------------------------------------------------------------------
// measured at top-10 of 512 (2048 -> 768 and 768 -> 2048): the down-shaped
// form (k <= 1024) wins from 64 tokens (1.25 pairs per expert) for IQ3_S and
// Q6_K and from 128 (2.5) for Q4_K; the gate/up-shaped form from 128 tokens
// for IQ3_S and Q4_K and from 64 for Q6_K
static int grouped_min_pairs(int form, int qt) {
    if (qt == QT_Q4_K) return 2;
    if (qt == QT_Q6_K) return 1;
    return form == 1 ? 1 : 2;
}
std::atomic<int> g_mmid_grouping{0};

SABAH_API int sabah_rt_set_mmid_grouping(int mode) {
    if (mode < 0 || mode > 2) return fail("MUL_MAT_ID grouping mode %d outside {0 auto, 1 never, 2 always}", mode);
    g_mmid_grouping.store(mode);
    return 0;
}

// the grouped kernels for the weight type qt (one of grouped_type_ok's)
static bool grouped_type_ok(int qt) { return qt == QT_IQ3_S || qt == QT_Q4_K || qt == QT_Q6_K; }

template <bool MMID>
static void launch_grouped_gate_up(int qt, int kind, dim3 grid, hipStream_t st, const GroupedGateUpArgs& a) {
    switch (qt) {
    case QT_Q4_K: launch_kernel(kind, k_grouped_gate_up<QT_Q4_K, MMID>, grid, dim3(kGuThreads), 0, st, a); break;
    case QT_Q6_K: launch_kernel(kind, k_grouped_gate_up<QT_Q6_K, MMID>, grid, dim3(kGuThreads), 0, st, a); break;
    default: launch_kernel(kind, k_grouped_gate_up<QT_IQ3_S, MMID>, grid, dim3(kGuThreads), 0, st, a); break;
    }
}

template <bool MMID, int ROWS>
static void launch_grouped_down_rows(int qt, int kind, dim3 grid, hipStream_t st, const GroupedDownArgs& a) {
    if constexpr (ROWS != kDownRows) {
        (void)qt;
        launch_kernel(kind, k_grouped_down<QT_Q4_K, MMID, ROWS>, grid, dim3(kThreads), 0, st, a);   // Q4_K only
    } else {
        switch (qt) {
        case QT_Q4_K: launch_kernel(kind, k_grouped_down<QT_Q4_K, MMID, ROWS>, grid, dim3(kThreads), 0, st, a); break;
        case QT_Q6_K: launch_kernel(kind, k_grouped_down<QT_Q6_K, MMID, ROWS>, grid, dim3(kThreads), 0, st, a); break;
        default: launch_kernel(kind, k_grouped_down<QT_IQ3_S, MMID, ROWS>, grid, dim3(kThreads), 0, st, a); break;
        }
    }
}
// rows: the output rows (a multiple of kDownRows).  Q4_K takes 128-row tiles
// where k <= 768 allows them (measured: a 512-token Q6_K / Q4_K layer 557
// against 590 us); IQ3_S measured slower with them (176 against 171 us per
// down launch) and Q6_K's would leave one workgroup per CU.
template <bool MMID>
static void launch_grouped_down(int qt, int kind, int rows, int n_experts, hipStream_t st, const GroupedDownArgs& a) {
    if (qt == QT_Q4_K && a.d_ff / 256 <= DownStage<QT_Q4_K, 2 * kDownRows>::NB && rows % (2 * kDownRows) == 0)
        launch_grouped_down_rows<MMID, 2 * kDownRows>(qt, kind, dim3((unsigned)(rows / (2 * kDownRows)), (unsigned)n_experts),
                                                      st, a);
    else
        launch_grouped_down_rows<MMID, kDownRows>(qt, kind, dim3((unsigned)(rows / kDownRows), (unsigned)n_experts), st, a);
}

// 0: not eligible; 1: down-shaped kernel (64-row tiles, k <= 1024); 2: gate/up-shaped (32-row tiles)
static int grouped_mmid_form(int qt, bool packed, size_t ids_id_stride, size_t ids_token_stride, size_t x_id_stride,
                             size_t x_token_stride, int x_rows, int n_ids, int n_tokens, int rows, int k,
                             int n_experts) {
    if (!grouped_type_ok(qt) || !packed || n_experts > 4096) return 0;
    if (ids_id_stride != 4 || ids_token_stride != 4 * (size_t)n_ids) return 0;
    if (x_id_stride != 4 * (size_t)k || x_token_stride != 4 * (size_t)k * x_rows) return 0;
    if ((size_t)n_tokens * n_ids > (size_t)1 << 24) return 0;
    if (k % 256 == 0 && k / 256 <= kDownBlocks && rows % kDownRows == 0) return 1;
    if (k % 512 == 0 && k / 256 <= kGuMaxBlocks && rows % (2 * kGuRows) == 0) return 2;
    return 0;
}

static int mmid_grouped(int form, int qt, const uint8_t* bank, size_t expert_stride, const float* d_x, int x_rows,
                        const int32_t* d_ids, int n_ids, int n_tokens, float* d_dst, size_t dst_id_stride,
                        size_t dst_token_stride, int rows, int k, int n_experts, hipStream_t st) {
    const size_t P = (size_t)n_tokens * n_ids;
    const int E = n_experts, nx = n_tokens * x_rows;
    const ActLayout XL(k, QT_Q8_K);
    const int xq_stride = (int)XL.bytes;
    int* off = static_cast<int*>(grow_scratch(g_scratch_goff, sizeof(int) * (size_t)(E + 1), st));
    int* pair_of = static_cast<int*>(grow_scratch(g_scratch_gpair, 2 * sizeof(int) * P, st));
    uint8_t* xq = static_cast<uint8_t*>(grow_scratch(g_scratch_gxq, (size_t)xq_stride * P, st));
    if (!off || !pair_of || !xq) return -1;
    int* pos_of = pair_of + P;
    GroupArgs ga{d_ids, n_tokens, n_ids, E, off, pair_of, pos_of, g_err_dev, d_dst, dst_id_stride, dst_token_stride, rows};
    // the grouping and quantisation launches time as part of the call
    // (KK_MMID), so a call's kernel time covers all three of its launches
    launch_kernel(KK_MMID, k_group_pairs, dim3(1), dim3(kGroupThreads), (int)sizeof(int) * (2 * E + kGroupThreads), st,
                  ga);
    // the pairs' x rows, quantised in group order (pair p = t * n_ids + s reads x row p / x_div)
    const int x_div = x_rows == 1 ? n_ids : 1;
    const size_t xq_rows = P * (size_t)(k / 256);
    launch_kernel(KK_MMID, k_quant_rows, dim3((unsigned)((xq_rows + 15) / 16)), dim3(kThreads), 0, st, d_x, (int)P, k,
                  (int)QT_Q8_K, xq, xq_stride, (const int*)pair_of, x_div, (const int*)(off + E), 1);
    (void)nx;
    if (form == 1) {
        GroupedDownArgs dn{};
        dn.down = bank;
        dn.expert_stride = expert_stride;
        dn.off = off;
        dn.hq = xq;
        dn.hq_stride = xq_stride;
        dn.d_model = rows;
        dn.d_ff = k;
        dn.pair_of = pair_of;
        dn.n_ids = n_ids;
        dn.dst = d_dst;
        dn.dst_nb1 = dst_id_stride;
        dn.dst_nb2 = dst_token_stride;
        launch_grouped_down<true>(qt, KK_MMID, rows, E, st, dn);
    } else {
        GroupedGateUpArgs gu{};
        gu.gate = bank;
        gu.expert_stride = expert_stride;
        gu.off = off;
        gu.pair_of = pair_of;
        gu.k = n_ids;
        gu.xq = xq;
        gu.xq_stride = xq_stride;
        gu.d_model = k;
        gu.d_ff = rows;
        gu.dst = d_dst;
        gu.dst_nb1 = dst_id_stride;
        gu.dst_nb2 = dst_token_stride;
        launch_grouped_gate_up<true>(qt, KK_MMID, dim3((unsigned)(rows / (2 * kGuRows)), (unsigned)E), st, gu);
    }
    return ck(hipGetLastError(), "grouped MUL_MAT_ID launch") ? 0 : -1;
}

static uint64_t mix64(uint64_t z) {   // splitmix64's finaliser
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// The self-check of one v2 call (see g_sc_k): waits for the stream, then
// recomputes min(k, n_tokens * n_ids) sampled (token, slot) output rows.  The
// samples are a hash of the call's number, never of its results.  Expert
// rows, inputs and outputs are copied from the device on the call's stream.
static void selfcheck_call(const uint8_t* bank, size_t expert_stride, size_t row_stride, const uint8_t* d_x,
                           size_t x_id_stride, int x_rows, size_t x_token_stride, const uint8_t* d_ids,
                           size_t ids_id_stride, size_t ids_token_stride, int n_ids, int n_tokens, const float* d_dst,
                           size_t dst_id_stride, size_t dst_token_stride, int rows, int k, int n_experts, int qt,
                           hipStream_t st) {
    const int K = g_sc_k.load();
    if (K <= 0) return;
    (void)hipStreamSynchronize(st);
    const uint64_t call_no = g_sc_calls++;
    const int sentinel = g_sc_sentinel.load();
    const size_t rb = row_bytes(qt, k);
    std::vector<float> x(k), out(rows), w(k);
    std::vector<uint8_t> wb((size_t)rows * row_stride);
    host::ActRow act;
    const int n_pairs = n_ids * n_tokens, samples = std::min(K, n_pairs);
    const uint64_t h0 = mix64(call_no * 0x9E3779B97F4A7C15ull + 0x5AB4ull);
    for (int smp = 0; smp < samples; ++smp) {
        const uint64_t h = mix64(h0 + (uint64_t)smp);
        int t = (int)(h % (uint64_t)n_tokens);
        int slot = (int)((mix64(h) + (uint64_t)smp) % (uint64_t)n_ids);
        int32_t e = 0;
        if (hipMemcpyAsync(&e, d_ids + (size_t)t * ids_token_stride + (size_t)slot * ids_id_stride, 4,
                           hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            ++g_sc_fail;
            continue;
        }
        if (e < 0 || e >= n_experts) continue;          // the kernel reports the id through the error word
        const int t_out = t, slot_out = slot;
        if (sentinel == 1) e = (e + 1) % n_experts;
        if (sentinel == 2) slot = (slot + 1) % n_ids;
        if (sentinel == 3) t = (t + 1) % n_tokens;
        const uint8_t* xp = d_x + (size_t)t * x_token_stride + (size_t)(slot % x_rows) * x_id_stride;
        const uint8_t* op = reinterpret_cast<const uint8_t*>(d_dst) + (size_t)t_out * dst_token_stride +
                            (size_t)slot_out * dst_id_stride;
        if (hipMemcpyAsync(x.data(), xp, (size_t)k * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipMemcpyAsync(out.data(), op, (size_t)rows * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipMemcpyAsync(wb.data(), bank + (size_t)e * expert_stride, wb.size(), hipMemcpyDeviceToHost, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            ++g_sc_fail;
            continue;
        }
        host::quantize_act(qt, x.data(), k, act);
        double num = 0.0, den = 0.0;
        for (int r = 0; r < rows; ++r) {
            const uint8_t* wr = wb.data() + (size_t)r * row_stride;
            host::dequant_row(qt, wr, w.data(), k);
            const double ref = host::ref_dot(qt, wr, w.data(), act, k);
            const double err = (double)out[r] - ref;
            num += err * err;
            den += ref * ref;
        }
        (void)rb;
        const double rel = den > 0.0 ? std::sqrt(num / den) : std::sqrt(num);
        std::lock_guard<std::mutex> lk(g_sc_mu);
        if (rel <= g_sc_tol) {
            ++g_sc_ok;
        } else {
            if (g_sc_fail.load() == 0)
                std::fprintf(stderr, "SABAH_SELFCHECK_FAIL call=%llu token=%d/%d slot=%d expert=%d rel_l2=%.3e\n",
                             (unsigned long long)call_no, t_out, n_tokens, slot_out, e, rel);
            ++g_sc_fail;
        }
        if (!(rel <= g_sc_max)) g_sc_max = rel;
    }
}

// SABAH_LLAMA_STATUS_FILE: the snapshot rewritten after every v2 call, before
// it returns (sabah_rt.cu:3418-3428), so a read after a request is exact.
static void write_status_file() {
    static const char* path = std::getenv("SABAH_LLAMA_STATUS_FILE");
    if (!path || !*path) return;
    char buf[1024];
    if (sabah_rt_snapshot(buf, sizeof(buf)) != 0) return;
    if (FILE* f = std::fopen(path, "wb")) {
        std::fputs(buf, f);
        std::fputc('\n', f);
        std::fclose(f);
    }
}

// SABAH_LLAMA_TRACE: the counters on stderr when the process exits
// (sabah_rt.cu:3096-3188)
static void report_trace_at_exit() {
    if (!std::getenv("SABAH_LLAMA_TRACE")) return;
    char buf[1024];
    if (sabah_rt_snapshot(buf, sizeof(buf)) == 0) std::fprintf(stderr, "SABAH_SNAPSHOT %s\n", buf);
    std::fprintf(stderr, "SABAH_DIAG calls=%llu tokens=%llu lookups=%llu overflow=0 verify_ok=%llu verify_fail=%llu\n",
                 g_calls.load(), g_tokens.load(), g_lookups.load(), g_sc_ok.load(), g_sc_fail.load());
}

// Harness control of the self-check (the environment sets it at init): k
// samples per call (0: off), the relative L2 tolerance, and the test-only
// perturbation of the recomputation (0 none, 1 expert, 2 slot row, 3 token row).
SABAH_API int sabah_rt_set_selfcheck(int k, double tol, int sentinel) {
    if (k < 0 || !(tol > 0.0) || sentinel < 0 || sentinel > 3)
        return fail("selfcheck: k %d >= 0, tol %g > 0 and sentinel %d in 0..3 expected", k, tol, sentinel);
    std::lock_guard<std::mutex> lk(g_sc_mu);
    g_sc_k.store(k);
    g_sc_tol = tol;
    g_sc_sentinel.store(sentinel);
    g_sc_ok.store(0);
    g_sc_fail.store(0);
    g_sc_max = 0.0;
    return 0;
}

SABAH_API int sabah_rt_mul_mat_id_v2(const void* source, size_t expert_stride, size_t row_stride, const void* d_x,
                                     size_t x_id_stride, int x_rows, size_t x_token_stride, const void* d_ids,
                                     size_t ids_id_stride, size_t ids_token_stride, int n_ids, int n_tokens,
                                     float* d_dst, size_t dst_id_stride, size_t dst_token_stride, int rows, int k,
                                     int n_experts, int qt, void* stream, const void* ids_key) {
    (void)ids_key;
    if (n_tokens == 0 && source && d_x && d_ids && d_dst) {
        // a graph may route zero token rows through an expert op (sabah_rt.cu:3520-3527)
        ++g_empty_calls;
        return 0;
    }
    if (validate_mmid(source, d_x, d_ids, d_dst, x_rows, n_ids, n_tokens, rows, k, n_experts, qt, row_stride))
        return -1;
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (!check_sticky()) return -1;
    const uint8_t* bank = resolve_source(source, expert_stride * (size_t)n_experts);
    if (!bank) return -1;
    hipStream_t st = pick_stream(stream);

    if (sync_ids_enabled()) {
        const size_t nb = (size_t)(n_ids - 1) * ids_id_stride + (size_t)(n_tokens - 1) * ids_token_stride + 4;
        std::vector<uint8_t> h(nb);
        if (!ck(hipMemcpyAsync(h.data(), d_ids, nb, hipMemcpyDeviceToHost, st), "ids download") ||
            !ck(hipStreamSynchronize(st), "ids download sync"))
            return -1;
        for (int t = 0; t < n_tokens; ++t)
            for (int i = 0; i < n_ids; ++i) {
                int32_t e;
                memcpy(&e, h.data() + (size_t)t * ids_token_stride + (size_t)i * ids_id_stride, 4);
                if (e < 0 || e >= n_experts) return fail("Sabah expert id out of range (token %d slot %d id %d)", t, i, e);
            }
    }

    const bool packed = row_stride == sabah_row_bytes(qt, k);
    const int mode = g_mmid_grouping.load();
    const int form = mode == 1 ? 0
                   : grouped_mmid_form(qt, packed, ids_id_stride, ids_token_stride, x_id_stride, x_token_stride,
                                       x_rows, n_ids, n_tokens, rows, k, n_experts);
    if (form && (mode == 2 || (long long)n_tokens * n_ids >= (long long)grouped_min_pairs(form, qt) * n_experts)) {
        if (mmid_grouped(form, qt, bank, expert_stride, static_cast<const float*>(d_x), x_rows,
                         static_cast<const int32_t*>(d_ids), n_ids, n_tokens, d_dst, dst_id_stride, dst_token_stride,
                         rows, k, n_experts, st))
            return -1;
        ++g_calls;
        ++g_grouped_calls;
        g_tokens += (unsigned long long)n_tokens;
        g_lookups += (unsigned long long)n_tokens * (unsigned long long)n_ids;
        selfcheck_call(bank, expert_stride, row_stride, static_cast<const uint8_t*>(d_x), x_id_stride, x_rows,
                       x_token_stride, static_cast<const uint8_t*>(d_ids), ids_id_stride, ids_token_stride, n_ids,
                       n_tokens, d_dst, dst_id_stride, dst_token_stride, rows, k, n_experts, qt, st);
        write_status_file();
        return 0;
    }

    MmidArgs a{};
    a.W.base = bank;
    a.W.ptrs = nullptr;
    a.W.expert_stride = expert_stride;
    a.rt.ids = reinterpret_cast<const uint8_t*>(d_ids);
    a.rt.id_stride = ids_id_stride;
    a.rt.token_stride = ids_token_stride;
    a.rt.n_experts = n_experts;
    a.row_stride = row_stride;
    a.x = reinterpret_cast<const uint8_t*>(d_x);
    a.x_id_stride = x_id_stride;
    a.x_token_stride = x_token_stride;
    a.x_rows = x_rows;
    a.n_ids = n_ids;
    a.n_tokens = n_tokens;
    a.dst = reinterpret_cast<uint8_t*>(d_dst);
    a.dst_id_stride = dst_id_stride;
    a.dst_token_stride = dst_token_stride;
    a.rows = rows;
    a.k = k;
    a.R = rows_mmid(qt, k, packed);
    if (packed)   // several tokens: longer row tiles in passes (as for the fused layer's kernels)
        a.R = grow_rows(a.R, rows, (long long)n_ids * n_tokens, kMaxPassesGateUp,
                        [&](int r) { return launch_lds(qt, make_plan(qt, k, 1, r * contribs_per_row(qt, k))); });
    a.err = g_err_dev;
    if (!ck(dispatch_mmid(qt, a, st), "MUL_MAT_ID launch")) return -1;
    ++g_calls;
    g_tokens += (unsigned long long)n_tokens;
    g_lookups += (unsigned long long)n_tokens * (unsigned long long)n_ids;
    selfcheck_call(bank, expert_stride, row_stride, static_cast<const uint8_t*>(d_x), x_id_stride, x_rows,
                   x_token_stride, static_cast<const uint8_t*>(d_ids), ids_id_stride, ids_token_stride, n_ids, n_tokens,
                   d_dst, dst_id_stride, dst_token_stride, rows, k, n_experts, qt, st);
    write_status_file();
    return 0;
}

// ===========================================================================
// observability
// ===========================================================================
static unsigned long long resident_bytes() {
    std::lock_guard<std::mutex> lk(g_mu);
    unsigned long long s = 0;
    for (const BankEntry& b : g_banks) s += b.bytes;
    return s;
}

SABAH_API int sabah_rt_get_metrics(unsigned long long* hits, unsigned long long* misses, unsigned long long* evictions,
                                   unsigned long long* bytes_fetched, unsigned long long* resident) {
    if (hits) *hits = g_lookups.load();
    if (misses) *misses = 0;
    if (evictions) *evictions = 0;
    if (bytes_fetched) *bytes_fetched = 0;
    if (resident) *resident = resident_bytes();
    return 0;
}

SABAH_API int sabah_rt_get_diag(unsigned long long* calls, unsigned long long* tokens, unsigned long long* overflow,
                                unsigned long long* verify_ok, unsigned long long* verify_fail) {
    if (calls) *calls = g_calls.load();
    if (tokens) *tokens = g_tokens.load();
    if (overflow) *overflow = 0;
    if (verify_ok) *verify_ok = g_sc_ok.load();         // self-check samples within / beyond tolerance
    if (verify_fail) *verify_fail = g_sc_fail.load();
    return 0;
}

SABAH_API int sabah_rt_snapshot(char* buf, size_t n) {
    if (!buf || n == 0) return fail("snapshot buffer is empty");
    double sc_max;
    {
        std::lock_guard<std::mutex> lk(g_sc_mu);
        sc_max = g_sc_max;
    }
    size_t nbanks;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        nbanks = g_banks.size();
    }
    const int w = snprintf(buf, n,
                           "{\"calls\":%llu,\"empty_calls\":%llu,\"tokens\":%llu,\"lookups\":%llu,\"hits\":%llu,"
                           "\"misses\":0,\"evictions\":0,\"bytes_fetched\":0,\"resident_bytes\":%llu,"
                           "\"banks\":%zu,\"layer_calls\":%llu,\"grouped_calls\":%llu,\"scratch_bytes\":%zu,"
                           "\"device\":%d,\"selfcheck_k\":%d,\"selfcheck_ok\":%llu,\"selfcheck_fail\":%llu,"
                           "\"selfcheck_max_rel\":%.3e,\"sentinel\":%d}",
                           g_calls.load(), g_empty_calls.load(), g_tokens.load(), g_lookups.load(), g_lookups.load(),
                           resident_bytes(), nbanks, g_layer_calls.load(), g_grouped_calls.load(), g_scratch_total,
                           g_device, g_sc_k.load(), g_sc_ok.load(), g_sc_fail.load(), sc_max, g_sc_sentinel.load());
    return (w < 0 || (size_t)w >= n) ? fail("snapshot buffer too small") : 0;
}

// ===========================================================================
// harness entry points
// ===========================================================================
SABAH_API size_t sabah_row_bytes(int qt, int n) { return supported_weight_type(qt) ? row_bytes(qt, n) : 0; }

SABAH_API int sabah_dequant(const void* d_src, float* d_dst, int qt, int n_rows, int row_elems) {
    if (!d_src || !d_dst || n_rows < 0) return fail("invalid dequant arguments");
    if (!supported_weight_type(qt) || row_bytes(qt, row_elems) == 0)
        return fail("dequant: unsupported type %d or row of %d elements", qt, row_elems);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (n_rows == 0) return 0;
    const long long nunits = (long long)n_rows * units_per_row(qt, row_elems);
    dim3 grid((unsigned)((nunits + kThreads - 1) / kThreads));
    const size_t lds = table_bytes(qt);
    const uint8_t* s = reinterpret_cast<const uint8_t*>(d_src);
    switch (qt) {
    case QT_Q8_0: hipLaunchKernelGGL(k_dequant<QT_Q8_0>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_Q4_K: hipLaunchKernelGGL(k_dequant<QT_Q4_K>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_Q5_K: hipLaunchKernelGGL(k_dequant<QT_Q5_K>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_Q5_1: hipLaunchKernelGGL(k_dequant<QT_Q5_1>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_Q6_K: hipLaunchKernelGGL(k_dequant<QT_Q6_K>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_IQ3_S: hipLaunchKernelGGL(k_dequant<QT_IQ3_S>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_IQ3_XXS: hipLaunchKernelGGL(k_dequant<QT_IQ3_XXS>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_IQ4_NL: hipLaunchKernelGGL(k_dequant<QT_IQ4_NL>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_Q2_0: hipLaunchKernelGGL(k_dequant<QT_Q2_0>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_IQ4_XS: hipLaunchKernelGGL(k_dequant<QT_IQ4_XS>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    case QT_IQ2_S: hipLaunchKernelGGL(k_dequant<QT_IQ2_S>, grid, dim3(kThreads), lds, g_stream, s, d_dst, n_rows, row_elems); break;
    }
    if (!ck(hipGetLastError(), "dequant launch")) return -1;
    return ck(hipStreamSynchronize(g_stream), "dequant sync") ? 0 : -1;
}

// n elements of type qt at host address src decoded on the host into n floats
// at dst (sabah_rt.cu:3845-3849): no GPU and no initialisation; the values are
// bit-identical to sabah_dequant's.
SABAH_API int sabah_rt_host_dequant(const void* src, float* dst, int qt, int n) {
    if (!src || !dst || n <= 0) return fail("invalid host dequant arguments");
    if (!host::dequant_row(qt, static_cast<const uint8_t*>(src), dst, n))
        return fail("host dequant: unsupported type %d or %d elements", qt, n);
    return 0;
}

SABAH_API int sabah_quantize_act(const float* d_x, void* d_y, int qt, int n_rows, int k, void* stream) {
    if (!d_x || !d_y || n_rows < 0) return fail("invalid quantize arguments");
    const int at = act_type(qt);
    if (at < 0 || k <= 0 || k % block_elems(at)) return fail("quantize: unsupported type %d or k=%d", qt, k);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (n_rows == 0) return 0;
    const size_t lds = ActLayout(k, at).bytes;
    hipLaunchKernelGGL(k_quantize_act_ggml, dim3((unsigned)n_rows), dim3(kThreads), lds, pick_stream(stream), d_x,
                       reinterpret_cast<uint8_t*>(d_y), k, at);
    return ck(hipGetLastError(), "quantize launch") ? 0 : -1;
}

// one layer on `st`: gate/up (+SwiGLU) -> h, then down + routed combine ->
// out; hq (or null) receives h quantised once per (token, slot) row
static int run_layer(const GateUpArgs& gu, int qtg, int qtd, const ExpertSrc& D, const Routing& rt, int n_slots,
                     int d_model, int d_ff, int n_tokens, const float* w, const float* shared, const float* resid,
                     float* out, int accumulate, uint8_t* hq, hipStream_t st, hipEvent_t join = nullptr) {
    if (!ck(dispatch_gate_up(qtg, gu, n_tokens, st), "gate/up launch")) return -1;
    DownArgs a{};
    a.D = D;
    a.rt = rt;
    a.h = gu.h;
    a.w = w;
    a.shared = shared;
    a.resid = resid;
    a.out = out;
    a.n_slots = n_slots;
    a.d_model = d_model;
    a.d_ff = d_ff;
    a.R = rows_down(qtd, d_ff, n_slots, d_model, n_tokens);
    a.accumulate = accumulate;
    a.err = g_err_dev;
    if (hq) {
        const int hb = down_hq_row_bytes(qtd, d_ff);
        const int n_rows = n_tokens * n_slots;
        const int chunk_rows = n_rows * (d_ff / 256);
        launch_kernel(KK_DOWN, k_quant_rows, dim3((unsigned)((chunk_rows + 15) / 16)), dim3(kThreads), 0, st, gu.h,
                      n_rows, d_ff, act_type(qtd), hq, hb, (const int*)nullptr, 1, (const int*)nullptr, 0);
        if (!ck(hipGetLastError(), "h quantisation launch")) return -1;
        a.hq = hq;
    }
    if (join && !ck(hipStreamWaitEvent(st, join, 0), "join the shared expert")) return -1;
    return ck(dispatch_down(qtd, a, n_tokens, st), "down/combine launch") ? 0 : -1;
}

// several tokens: h is quantised once per (token, slot) row rather than in
// every down workgroup (one launch; a single token keeps the fused form)
static bool layer_quantises_h_once(int qtd, int d_ff, int n_slots, int n_tokens) {
    return n_tokens >= 2 && down_hq_fits(qtd, d_ff, n_slots) && d_ff % 256 == 0;
}

static bool layer_types_ok(int qtg, int qtu, int qtd, int d_model, int d_ff) {
    if (!supported_weight_type(qtg) || !supported_weight_type(qtu) || !supported_weight_type(qtd)) return false;
    if (qtg != qtu) return false;   // gate and up share one fused kernel instantiation
    return row_bytes(qtg, d_model) && row_bytes(qtd, d_ff);
}

SABAH_API int sabah_moe_block(const float* d_x, float* d_out, float* d_h, const void* const* d_ptrs, const float* d_w,
                              int d_model, int ff, int n_used, int qt_gate, int qt_up, int qt_down, int accumulate) {
    if (!d_x || !d_out || !d_h || !d_ptrs || !d_w || n_used <= 0) return fail("invalid moe_block arguments");
    if (n_used > kMaxTiles) return fail("n_used %d exceeds the supported maximum %d", n_used, kMaxTiles);
    if ((d_model % 32) || (ff % 32)) return fail("d_model and ff must be multiples of 32");
    if (!layer_types_ok(qt_gate, qt_up, qt_down, d_model, ff))
        return fail("moe_block: unsupported type mix gate=%d up=%d down=%d", qt_gate, qt_up, qt_down);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    GateUpArgs gu{};
    gu.G = {nullptr, d_ptrs, 0};
    gu.U = {nullptr, d_ptrs + n_used, 0};
    gu.rt = {nullptr, 0, 0, 0};
    gu.x = d_x;
    gu.h = d_h;
    gu.n_slots = n_used;
    gu.d_model = d_model;
    gu.d_ff = ff;
    gu.R = rows_gate_up(qt_gate, d_model, ff, n_used, 1);
    gu.err = g_err_dev;
    const ExpertSrc D{nullptr, d_ptrs + 2 * n_used, 0};
    ++g_layer_calls;
    return run_layer(gu, qt_gate, qt_down, D, gu.rt, n_used, d_model, ff, 1, d_w, nullptr, nullptr, d_out, accumulate,
                     nullptr, g_stream);
}

// Device scratch of a layer call: h, the shared expert's hs and ys, and the
// several-token q8 rows of h.  A Workspace hands them out either from the
// library's grow-only buffers (arena null) or from a fixed arena, carved
// front to back at 256-byte alignment.
struct LayerBufs {
    float *h = nullptr, *hs = nullptr, *ys = nullptr;
    uint8_t* hq = nullptr;
    uint8_t *sxq = nullptr, *shq = nullptr;   // the shared expert's quantised x and h (several tokens)
    float* sgl = nullptr;                     // its gate logits
};
struct Workspace {
    uint8_t* arena = nullptr;
    size_t cap = 0, used = 0;
    void* get(Scratch& s, size_t bytes, hipStream_t st) {
        if (!arena) return grow_scratch(s, bytes, st);
        const size_t off = (used + 255) & ~(size_t)255;
        if (off + bytes > cap) return nullptr;   // callers check the total first (layer_scratch_bytes)
        used = off + bytes;
        return arena + off;
    }
};
// The shared expert over at least this many tokens reads each weight row once
// per launch (k_dense_tokens) instead of once per token.
constexpr int kDenseMinTokens = 4;
constexpr int kDenseMaxTB = 32;                 // tokens per workgroup
// quantised activation row stride: the ActLayout, then 16 bytes, so the
// same offset of consecutive tokens' rows falls on different LDS banks
static int dense_act_stride(int qt, int k) { return align16i((int)ActLayout(k, act_type(qt)).bytes) + 16; }
static bool shared_dense(const sabah_moe_layer_desc* L, int n_tokens) {
    return L->shared_gate && n_tokens >= kDenseMinTokens && L->qt_shared_gate == L->qt_shared_up &&
           L->d_model % 256 == 0 && L->d_ff_shared % 256 == 0;
}
static size_t layer_hq_bytes(const sabah_moe_layer_desc* L, int n_used, int n_tokens) {
    if (!layer_quantises_h_once(L->qt_down, L->d_ff, n_used, n_tokens)) return 0;
    return (size_t)down_hq_row_bytes(L->qt_down, L->d_ff) * n_tokens * n_used;
}
// bytes a Workspace arena must hold for one layer call (the same requests,
// in the same order and alignment, as layer_bufs makes)
static size_t layer_scratch_bytes(const sabah_moe_layer_desc* L, int n_used, int n_tokens) {
    size_t used = 0;
    auto take = [&](size_t b) { used = ((used + 255) & ~(size_t)255) + b; };
    if (L->shared_gate) {
        take(sizeof(float) * (size_t)n_tokens * L->d_ff_shared);
        take(sizeof(float) * (size_t)n_tokens * L->d_model);
    }
    if (shared_dense(L, n_tokens)) {
        take((size_t)n_tokens * dense_act_stride(L->qt_shared_gate, L->d_model));
        take((size_t)n_tokens * dense_act_stride(L->qt_shared_down, L->d_ff_shared));
        take(sizeof(float) * (size_t)n_tokens);
    }
    take(sizeof(float) * (size_t)n_tokens * n_used * L->d_ff);
    if (const size_t hq = layer_hq_bytes(L, n_used, n_tokens)) take(hq);
    return used;
}
static int layer_bufs(const sabah_moe_layer_desc* L, int n_used, int n_tokens, Workspace& ws, hipStream_t st,
                      LayerBufs& b) {
    if (L->shared_gate) {
        b.hs = static_cast<float*>(ws.get(g_scratch_hs, sizeof(float) * (size_t)n_tokens * L->d_ff_shared, st));
        b.ys = static_cast<float*>(ws.get(g_scratch_ys, sizeof(float) * (size_t)n_tokens * L->d_model, st));
        if (!b.hs || !b.ys) return -1;
    }
    if (shared_dense(L, n_tokens)) {
        b.sxq = static_cast<uint8_t*>(
            ws.get(g_scratch_sxq, (size_t)n_tokens * dense_act_stride(L->qt_shared_gate, L->d_model), st));
        b.shq = static_cast<uint8_t*>(
            ws.get(g_scratch_shq, (size_t)n_tokens * dense_act_stride(L->qt_shared_down, L->d_ff_shared), st));
        b.sgl = static_cast<float*>(ws.get(g_scratch_sgl, sizeof(float) * (size_t)n_tokens, st));
        if (!b.sxq || !b.shq || !b.sgl) return -1;
    }
    b.h = static_cast<float*>(ws.get(g_scratch_h, sizeof(float) * (size_t)n_tokens * n_used * L->d_ff, st));
    if (!b.h) return -1;
    if (const size_t hq = layer_hq_bytes(L, n_used, n_tokens)) {
        b.hq = static_cast<uint8_t*>(ws.get(g_scratch_hq, hq, st));
        if (!b.hq) return -1;
    }
    return 0;
}

// dense shared expert of a layer: gate/up + SwiGLU -> hs, down -> ys (added
// by the routed combine); nothing when the layer has none
template <int QT, int NMAT>
hipError_t launch_dense(const DenseArgs& a, int kind, hipStream_t st) {
    const int dyn = dense_dyn_lds(a.TB, a.act_stride, NMAT, a.R);
    if (const hipError_t e = fit_lds(k_dense_tokens<QT, NMAT>, dyn, StaticLds<QT>::BYTES + dyn)) return e;
    const dim3 grid((unsigned)((a.rows + a.R - 1) / a.R), (unsigned)((a.n_tokens + a.TB - 1) / a.TB));
    launch_kernel(kind, k_dense_tokens<QT, NMAT>, grid, dim3(kThreads), dyn, st, a);
    return hipGetLastError();
}
template <int NMAT>
hipError_t dispatch_dense(int qt, const DenseArgs& a, int kind, hipStream_t st) {
    switch (qt) {
    case QT_Q8_0: return launch_dense<QT_Q8_0, NMAT>(a, kind, st);
    case QT_Q4_K: return launch_dense<QT_Q4_K, NMAT>(a, kind, st);
    case QT_Q5_K: return launch_dense<QT_Q5_K, NMAT>(a, kind, st);
    case QT_Q5_1: return launch_dense<QT_Q5_1, NMAT>(a, kind, st);
    case QT_Q6_K: return launch_dense<QT_Q6_K, NMAT>(a, kind, st);
    case QT_IQ3_S: return launch_dense<QT_IQ3_S, NMAT>(a, kind, st);
    case QT_IQ3_XXS: return launch_dense<QT_IQ3_XXS, NMAT>(a, kind, st);
    case QT_IQ4_NL: return launch_dense<QT_IQ4_NL, NMAT>(a, kind, st);
    case QT_Q2_0: return launch_dense<QT_Q2_0, NMAT>(a, kind, st);
    case QT_IQ4_XS: return launch_dense<QT_IQ4_XS, NMAT>(a, kind, st);
    case QT_IQ2_S: return launch_dense<QT_IQ2_S, NMAT>(a, kind, st);
    }
    return hipErrorInvalidValue;
}

// Tokens and rows per workgroup of a dense launch: up to kDenseMaxTB tokens,
// one thread per (token, matrix, row), the tiles staged in one pass, the
// activation rows within kDenseActLoads loads per thread and the LDS limit.
static bool dense_shape(int qt, int k, int n_mat, int n_tokens, int act_stride, int& R, int& TB) {
    const int rmax = std::max(1, (16 * tile_chunk_cap(qt, n_mat) - 30) / (int)row_bytes(qt, k));
    for (TB = std::min(n_tokens, kDenseMaxTB); TB >= 1; TB = TB > 1 ? (TB + 1) / 2 : 0) {
        R = std::min(rmax, kThreads / (TB * n_mat));
        if (R < 1) continue;
        const int lds = table_bytes(qt) + 4 * kMaxTiles + 2 * kStageGuard + kStageBytes +
                        dense_dyn_lds(TB, act_stride, n_mat, R) + 64;
        if (TB * act_stride <= 16 * kThreads * kDenseActLoads && lds <= g_max_lds) return true;
        if (TB == 1) break;
    }
    return false;
}

// The shared expert over n_tokens >= kDenseMinTokens: x quantised once, gate/up
// + SwiGLU with every weight row read once per kDenseMaxTB tokens (and the gate
// logits), h quantised once, down scaled by the gate.  The same values as the
// token-major launches, bit for bit.
static int shared_expert_dense(const sabah_moe_layer_desc* L, const float* d_x, int n_tokens, float* hs, float* ys,
                               uint8_t* sxq, uint8_t* shq, float* sgl, hipStream_t st) {
    const int D = L->d_model, Fs = L->d_ff_shared;
    const int qg = L->qt_shared_gate, qd = L->qt_shared_down;
    DenseArgs g{};
    g.act_stride = dense_act_stride(qg, D);
    DenseArgs d{};
    d.act_stride = dense_act_stride(qd, Fs);
    if (!dense_shape(qg, D, 2, n_tokens, g.act_stride, g.R, g.TB) ||
        !dense_shape(qd, Fs, 1, n_tokens, d.act_stride, d.R, d.TB))
        return 1;                                            // the token-major launches then
    const size_t xrows = (size_t)n_tokens * (D / 256);
    launch_kernel(KK_GATE_UP, k_quant_rows, dim3((unsigned)((xrows + 15) / 16)), dim3(kThreads), 0, st, d_x,
                  n_tokens, D, act_type(qg), sxq, g.act_stride, (const int*)nullptr, 1, (const int*)nullptr, 0);
    g.w0 = static_cast<const uint8_t*>(L->shared_gate);
    g.w1 = static_cast<const uint8_t*>(L->shared_up);
    g.xq = sxq;
    g.n_tokens = n_tokens;
    g.k = D;
    g.rows = Fs;
    g.out = hs;
    g.sg_w = L->shared_gate_inp;
    g.sg_x = d_x;
    g.sg_n = D;
    g.sg_logit = sgl;
    if (!ck(dispatch_dense<2>(qg, g, KK_GATE_UP, st), "shared gate/up launch")) return -1;
    const size_t hrows = (size_t)n_tokens * (Fs / 256);
    launch_kernel(KK_MMID, k_quant_rows, dim3((unsigned)((hrows + 15) / 16)), dim3(kThreads), 0, st,
                  (const float*)hs, n_tokens, Fs, act_type(qd), shq, d.act_stride, (const int*)nullptr, 1,
                  (const int*)nullptr, 0);
    d.w0 = static_cast<const uint8_t*>(L->shared_down);
    d.w1 = nullptr;
    d.xq = shq;
    d.n_tokens = n_tokens;
    d.k = Fs;
    d.rows = D;
    d.out = ys;
    d.sg_logit = L->shared_gate_inp ? sgl : nullptr;
    return ck(dispatch_dense<1>(qd, d, KK_MMID, st), "shared down launch") ? 0 : -1;
}

static int shared_expert(const sabah_moe_layer_desc* L, const float* d_x, int n_tokens, float* hs, float* ys,
                         hipStream_t st, uint8_t* sxq = nullptr, uint8_t* shq = nullptr, float* sgl = nullptr) {
    if (!L->shared_gate) return 0;
    if (sxq && shared_dense(L, n_tokens)) {
        const int rc = shared_expert_dense(L, d_x, n_tokens, hs, ys, sxq, shq, sgl, st);
        if (rc <= 0) return rc;
    }
    const int D = L->d_model;
    const int Fs = L->d_ff_shared;
    GateUpArgs gs{};
    gs.G = {reinterpret_cast<const uint8_t*>(L->shared_gate), nullptr, 0};
    gs.U = {reinterpret_cast<const uint8_t*>(L->shared_up), nullptr, 0};
    gs.rt = {nullptr, 0, 0, 1};
    gs.x = d_x;
    gs.h = hs;
    gs.n_slots = 1;
    gs.d_model = D;
    gs.d_ff = Fs;
    gs.R = rows_gate_up(L->qt_shared_gate, D, Fs, 1, 1);   // single-pass tiles: grown ones ran slower here
    gs.err = g_err_dev;
    if (!ck(dispatch_gate_up(L->qt_shared_gate, gs, n_tokens, st), "shared gate/up launch")) return -1;
    MmidArgs a{};
    a.W = {reinterpret_cast<const uint8_t*>(L->shared_down), nullptr, 0};
    a.rt = {nullptr, 0, 0, 1};
    a.row_stride = row_bytes(L->qt_shared_down, Fs);
    a.x = reinterpret_cast<const uint8_t*>(hs);
    a.x_id_stride = (size_t)Fs * 4;
    a.x_token_stride = (size_t)Fs * 4;
    a.x_rows = 1;
    a.n_ids = 1;
    a.n_tokens = n_tokens;
    a.dst = reinterpret_cast<uint8_t*>(ys);
    a.dst_id_stride = (size_t)D * 4;
    a.dst_token_stride = (size_t)D * 4;
    a.rows = D;
    a.k = Fs;
    a.R = rows_mmid(L->qt_shared_down, Fs, true);
    a.err = g_err_dev;
    a.sg_w = L->shared_gate_inp;                 // ggml_mul(ffn_shexp, sigmoid(gate_inp_shexp . x))
    a.sg_x = d_x;
    a.sg_n = D;
    return ck(dispatch_mmid(L->qt_shared_down, a, st), "shared down launch") ? 0 : -1;
}

// The fused layer's down workgroups wait this long (10 ns ticks) before their
// weight loads: the time the gate/up weights take at 7.5 TB/s (75,000 bytes
// per tick), so the gate/up bytes, needed first, are not shared with them.
// On the 48-layer decode (13.5 MB of gate/up weights, 180 ticks) the layer
// measured 11.7 us against 12.7 us without the wait (per-workgroup stamps,
// same box, interleaved launches); 150-200 ticks were best.
static uint32_t layer_down_delay(int qt, int n_used, int D, int F) {
    const size_t g_bytes = (size_t)n_used * 2 * F * row_bytes(qt, D);
    return (uint32_t)std::min<size_t>(g_bytes / 75000, 1000);
}

// The layer's lockstep arguments for a fused launch (the flags cleared first
// when an earlier wait ran out)
static LayerArgs layer_args(const GateUpArgs& gu, const DownArgs& dn, int qt, int n_g, int g_tiles, int n_d,
                            hipStream_t st) {
    uint32_t* sync = g_layer_sync[g_device];
    if (g_sync_reset_pending.exchange(false)) launch_kernel(KK_LAYER, k_clear_sync, dim3(1), dim3(256), 0, st, sync);
    const bool wait_test = g_layer_wait_test.exchange(false);
    // the timeout test gives up after 2 ms without progress rather than 50
    return LayerArgs{gu, dn, n_g, g_tiles, n_d, sync, wait_test ? 1u : 0u,
                     layer_down_delay(qt, dn.n_slots, dn.d_model, dn.d_ff),
                     wait_test ? 200000u : (uint32_t)kLayerIdleTicks, g_layer_xcd_groups.load()};
}

// A one-token IQ3_S layer as one launch (k_layer_decode) when it applies:
// returns 1 when launched, 0 when the two-kernel form must run, -1 on error.
// (The same fusion for Q8_0 / Q4_K / Q5_K / Q6_K layers, down rows staged in
// one pass before the wait, measured slower than their two kernels on the
// 1-token Q8_0 E=8 and Q4_K E=128 layers: 12.1 against 11.4 us and 15.4
// against 13.0 us per layer; there the hand-over costs more than the
// second launch and the down weights' load it would hide.)
static int layer_fused(const sabah_moe_layer_desc* L, const GateUpArgs& gu, const ExpertSrc& DS, const Routing& rt,
                       int n_used, const float* w, const float* shared, const float* resid, float* out,
                       hipStream_t st) {
    constexpr int QT = QT_IQ3_S;
    if (!g_layer_fusion.load() || g_device < 0 || g_device >= kMaxDevices || !g_layer_sync[g_device]) return 0;
    const int D = L->d_model, F = L->d_ff;
    DownArgs dn{};
    dn.D = DS;
    dn.rt = rt;
    dn.h = gu.h;
    dn.w = w;
    dn.shared = shared;
    dn.resid = resid;
    dn.out = out;
    dn.n_slots = n_used;
    dn.d_model = D;
    dn.d_ff = F;
    dn.err = g_err_dev;
    if (L->qt_gate != QT || L->qt_up != QT || L->qt_down != QT) return 0;
    if (!gate_up_rounds_ok(QT, D) || gu.R != rows_gate_up_rounds(QT, D) || F % 256) return 0;
    static_assert(GateUpRounds<QT, kLayerThreads, 2>::STAGE <= kStageBytes, "gate/up rounds stage in the static area");
    dn.R = rows_down(QT, F, n_used, D, 1);
    const int g_tiles = (F + gu.R - 1) / gu.R;
    const int n_g = g_tiles * n_used, n_d = (D + dn.R - 1) / dn.R;
    if (n_g > kSyncG || n_d > kSyncD) return 0;
    // the down workgroup's tiles stage in one pass (TileWalk's pass size at kLayerThreads threads)
    const int cap = std::min(kStageChunks / n_used, stage_iters_nt(QT, kLayerThreads) * (kLayerThreads / n_used));
    if (dn.R * units_per_row(QT, F) > std::max(1, (16 * cap - 30) / UnitFmt<QT>::BYTES)) return 0;
    // at most one unit per lane pair: each lane holds its decoded half unit
    if (n_used * dn.R * units_per_row(QT, F) > kLayerThreads / 2) return 0;
    const int dyn = layer_dyn_lds(gu, dn);
    if (StaticLds<QT>::BYTES + dyn + 64 > g_max_lds) return 0;
    if (!ck(fit_lds(k_layer_decode<kLayerThreads>, dyn, StaticLds<QT>::BYTES + dyn), "fused layer LDS")) return -1;
    const LayerArgs a = layer_args(gu, dn, QT, n_g, g_tiles, n_d, st);
    launch_kernel(KK_LAYER, k_layer_decode<kLayerThreads>, dim3((unsigned)(n_g + n_d)), dim3(kLayerThreads), dyn, st, a);
    return ck(hipGetLastError(), "fused layer launch") ? 1 : -1;
}

// The batched shared expert on g_side: the fork (an event of the caller's
// stream the side stream waits for), its launches, and the join event
// recorded after them.  Called with g_side_mu held.
static int shared_expert_forked(const sabah_moe_layer_desc* L, const float* d_x, int n_tokens, float* hs, float* ys,
                                uint8_t* sxq, uint8_t* shq, float* sgl, hipStream_t st) {
    if (!ck(hipEventRecord(g_ev_fork, st), "fork the shared expert") ||
        !ck(hipStreamWaitEvent(g_side, g_ev_fork, 0), "fork the shared expert"))
        return -1;
    if (shared_expert(L, d_x, n_tokens, hs, ys, g_side, sxq, shq, sgl)) return -1;
    return ck(hipEventRecord(g_ev_join, g_side), "join the shared expert") ? 0 : -1;
}
// the batches whose shared expert overlaps the routed experts (the batched
// shared expert's own launches then run beside the routed gate/up)
static bool shared_overlaps(const sabah_moe_layer_desc* L, int n_tokens) { return g_side && shared_dense(L, n_tokens); }

static int moe_layer_on(const sabah_moe_layer_desc* L, const float* d_x, const int32_t* d_ids, const float* d_w,
                        int n_used, int n_tokens, float* d_out, const float* d_resid, Workspace& ws, hipStream_t st) {
    const int D = L->d_model, F = L->d_ff;
    LayerBufs b;
    if (layer_bufs(L, n_used, n_tokens, ws, st, b)) return -1;
    std::unique_lock<std::mutex> side_lock(g_side_mu, std::defer_lock);
    hipEvent_t join = nullptr;
    if (shared_overlaps(L, n_tokens)) {
        side_lock.lock();
        if (shared_expert_forked(L, d_x, n_tokens, b.hs, b.ys, b.sxq, b.shq, b.sgl, st)) return -1;
        join = g_ev_join;
    } else if (shared_expert(L, d_x, n_tokens, b.hs, b.ys, st, b.sxq, b.shq, b.sgl)) {
        return -1;
    }
    const Routing rt{reinterpret_cast<const uint8_t*>(d_ids), 4, (size_t)n_used * 4, L->n_experts};
    GateUpArgs gu{};
    gu.G = {reinterpret_cast<const uint8_t*>(L->gate), nullptr, row_bytes(L->qt_gate, D) * (size_t)F};
    gu.U = {reinterpret_cast<const uint8_t*>(L->up), nullptr, row_bytes(L->qt_up, D) * (size_t)F};
    gu.rt = rt;
    gu.x = d_x;
    gu.h = b.h;
    gu.n_slots = n_used;
    gu.d_model = D;
    gu.d_ff = F;
    gu.R = rows_gate_up(L->qt_gate, D, F, n_used, n_tokens);
    gu.err = g_err_dev;
    const ExpertSrc DS{reinterpret_cast<const uint8_t*>(L->down), nullptr, row_bytes(L->qt_down, F) * (size_t)D};
    if (n_tokens == 1) {
        const int f = layer_fused(L, gu, DS, rt, n_used, d_w, b.ys, d_resid, d_out, st);
        if (f) return f > 0 ? 0 : -1;
    }
    return run_layer(gu, L->qt_gate, L->qt_down, DS, rt, n_used, D, F, n_tokens, d_w, b.ys, d_resid, d_out, 0, b.hq,
                     st, join);
}

static int check_layer_desc(const sabah_moe_layer_desc* L) {
    if (!L || !L->gate || !L->up || !L->down || L->n_experts <= 0) return fail("invalid MoE layer descriptor");
    if (!layer_types_ok(L->qt_gate, L->qt_up, L->qt_down, L->d_model, L->d_ff))
        return fail("MoE layer: unsupported type mix gate=%d up=%d down=%d (d_model=%d d_ff=%d)", L->qt_gate,
                    L->qt_up, L->qt_down, L->d_model, L->d_ff);
    if (L->shared_gate) {
        if (!L->shared_up || !L->shared_down || L->d_ff_shared <= 0 ||
            !layer_types_ok(L->qt_shared_gate, L->qt_shared_up, L->qt_shared_down, L->d_model, L->d_ff_shared))
            return fail("MoE layer: invalid shared expert");
    } else if (L->shared_gate_inp) {
        return fail("MoE layer: shared_gate_inp given without a shared expert");
    }
    return 0;
}

SABAH_API int sabah_moe_layer(const sabah_moe_layer_desc* layer, const float* d_x, const int32_t* d_ids,
                              const float* d_w, int n_used, int n_tokens, float* d_out, const float* d_resid,
                              void* stream) {
    if (check_layer_desc(layer)) return -1;
    if (!d_x || !d_ids || !d_w || !d_out || n_used <= 0 || n_tokens < 0) return fail("invalid MoE layer arguments");
    if (n_used > kMaxTiles) return fail("n_used %d exceeds the supported maximum %d", n_used, kMaxTiles);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (!check_sticky()) return -1;
    if (n_tokens == 0) return 0;
    ++g_layer_calls;
    g_lookups += (unsigned long long)n_tokens * n_used;
    Workspace ws;
    return moe_layer_on(layer, d_x, d_ids, d_w, n_used, n_tokens, d_out, d_resid, ws, pick_stream(stream));
}

// sabah_moe_layer with all of its device scratch in the library's static
// array (8 MiB per GPU): no allocation of any kind, so it may be called
// where allocating is not allowed (stream capture, serving loops).  Calls on
// one GPU share the array: calls that overlap on different streams race.
SABAH_API int sabah_moe_layer_noalloc(const sabah_moe_layer_desc* layer, const float* d_x, const int32_t* d_ids,
                                      const float* d_w, int n_used, int n_tokens, float* d_out, const float* d_resid,
                                      void* stream) {
    if (check_layer_desc(layer)) return -1;
    if (!d_x || !d_ids || !d_w || !d_out || n_used <= 0 || n_tokens < 0) return fail("invalid MoE layer arguments");
    if (n_used > kMaxTiles) return fail("n_used %d exceeds the supported maximum %d", n_used, kMaxTiles);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (!check_sticky()) return -1;
    if (n_tokens == 0) return 0;
    const size_t need = layer_scratch_bytes(layer, n_used, n_tokens);
    if (need > kNoAllocScratchBytes)
        return fail("sabah_moe_layer_noalloc: %d tokens x %d experts (d_ff %d) need %zu bytes of scratch, more "
                    "than the %zu bytes of its static scratch; split the tokens or call sabah_moe_layer",
                    n_tokens, n_used, layer->d_ff, need, kNoAllocScratchBytes);
    if (g_device >= kMaxDevices || !g_noalloc_scratch[g_device])
        return fail("sabah_moe_layer_noalloc: no static scratch on device %d", g_device);
    ++g_layer_calls;
    g_lookups += (unsigned long long)n_tokens * n_used;
    Workspace ws;
    ws.arena = static_cast<uint8_t*>(g_noalloc_scratch[g_device]);
    ws.cap = kNoAllocScratchBytes;
    g_launch_plain = true;
    const int rc = moe_layer_on(layer, d_x, d_ids, d_w, n_used, n_tokens, d_out, d_resid, ws, pick_stream(stream));
    g_launch_plain = false;
    return rc;
}

SABAH_API int sabah_moe_chain(const sabah_moe_layer_desc* layers, int n_layers, float* d_x, const int32_t* d_ids,
                              const float* d_w, int n_used, int n_tokens, void* stream) {
    if (!layers || n_layers <= 0 || !d_x || !d_ids || !d_w || n_used <= 0 || n_tokens < 0)
        return fail("invalid MoE chain arguments");
    if (n_used > kMaxTiles) return fail("n_used %d exceeds the supported maximum %d", n_used, kMaxTiles);
    for (int l = 0; l < n_layers; ++l)
        if (check_layer_desc(layers + l)) return -1;
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (!check_sticky()) return -1;
    if (n_tokens == 0) return 0;
    hipStream_t st = pick_stream(stream);
    const size_t per = (size_t)n_tokens * n_used;
    for (int l = 0; l < n_layers; ++l) {
        Workspace ws;
        if (moe_layer_on(layers + l, d_x, d_ids + per * l, d_w + per * l, n_used, n_tokens, d_x, d_x, ws, st))
            return -1;
    }
    g_layer_calls += (unsigned long long)n_layers;
    g_lookups += (unsigned long long)n_layers * per;
    return 0;
}

// ===========================================================================
// group-major layer for a batch of tokens (prefill)
// ===========================================================================
static bool grouped_shape_ok(const sabah_moe_layer_desc* L) {
    const int D = L->d_model, F = L->d_ff;
    return grouped_type_ok(L->qt_gate) && L->qt_up == L->qt_gate && grouped_type_ok(L->qt_down) && D % 512 == 0 &&
           D / 256 <= kGuMaxBlocks && F % 256 == 0 && F / 256 <= kDownBlocks && D % kDownRows == 0 &&
           L->n_experts <= 4096;
}

static int moe_prefill_on(const sabah_moe_layer_desc* L, const float* d_x, const int32_t* d_ids, const float* d_w,
                          int n_used, int n_tokens, float* d_out, const float* d_resid, hipStream_t st) {
    const int D = L->d_model, F = L->d_ff, E = L->n_experts;
    const size_t P = (size_t)n_tokens * n_used;
    const ActLayout XL(D, QT_Q8_K), HL(F, QT_Q8_K);
    const int xq_stride = (int)XL.bytes, hq_stride = (int)HL.bytes;
    int* off = static_cast<int*>(grow_scratch(g_scratch_goff, sizeof(int) * (size_t)(E + 1), st));
    int* pair_of = static_cast<int*>(grow_scratch(g_scratch_gpair, 2 * sizeof(int) * P, st));
    uint8_t* xq = static_cast<uint8_t*>(grow_scratch(g_scratch_gxq, (size_t)xq_stride * P, st));
    float* h = static_cast<float*>(grow_scratch(g_scratch_gh, sizeof(float) * P * F, st));
    uint8_t* hq = static_cast<uint8_t*>(grow_scratch(g_scratch_ghq, (size_t)hq_stride * P, st));
    float* y = static_cast<float*>(grow_scratch(g_scratch_gy, sizeof(float) * P * D, st));
    if (!off || !pair_of || !xq || !h || !hq || !y) return -1;
    int* pos_of = pair_of + P;
    float *hs = nullptr, *shared = nullptr, *sgl = nullptr;
    uint8_t *sxq = nullptr, *shq = nullptr;
    if (L->shared_gate) {
        hs = static_cast<float*>(grow_scratch(g_scratch_hs, sizeof(float) * (size_t)n_tokens * L->d_ff_shared, st));
        shared = static_cast<float*>(grow_scratch(g_scratch_ys, sizeof(float) * (size_t)n_tokens * D, st));
        if (!hs || !shared) return -1;
    }
    if (shared_dense(L, n_tokens)) {
        sxq = static_cast<uint8_t*>(
            grow_scratch(g_scratch_sxq, (size_t)n_tokens * dense_act_stride(L->qt_shared_gate, D), st));
        shq = static_cast<uint8_t*>(
            grow_scratch(g_scratch_shq, (size_t)n_tokens * dense_act_stride(L->qt_shared_down, L->d_ff_shared), st));
        sgl = static_cast<float*>(grow_scratch(g_scratch_sgl, sizeof(float) * (size_t)n_tokens, st));
        if (!sxq || !shq || !sgl) return -1;
    }
    std::unique_lock<std::mutex> side_lock(g_side_mu, std::defer_lock);
    hipEvent_t join = nullptr;
    if (shared_overlaps(L, n_tokens)) {
        side_lock.lock();
        if (shared_expert_forked(L, d_x, n_tokens, hs, shared, sxq, shq, sgl, st)) return -1;
        join = g_ev_join;
    } else if (shared_expert(L, d_x, n_tokens, hs, shared, st, sxq, shq, sgl)) {
        return -1;
    }

    GroupArgs ga{d_ids, n_tokens, n_used, E, off, pair_of, pos_of, g_err_dev, nullptr, 0, 0, 0};
    hipLaunchKernelGGL(k_group_pairs, dim3(1), dim3(kGroupThreads), sizeof(int) * (2 * E + kGroupThreads), st, ga);
    // the pairs' x rows in group order (pair p is token p / n_used)
    const size_t xq_rows = P * (size_t)(D / 256);
    hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((xq_rows + 15) / 16)), dim3(kThreads), 0, st, d_x, (int)P, D,
                       (int)QT_Q8_K, xq, xq_stride, (const int*)pair_of, n_used, (const int*)(off + E), 1);
    GroupedGateUpArgs gu{};
    gu.gate = static_cast<const uint8_t*>(L->gate);
    gu.up = static_cast<const uint8_t*>(L->up);
    gu.expert_stride = row_bytes(L->qt_gate, D) * (size_t)F;
    gu.off = off;
    gu.pair_of = pair_of;
    gu.k = n_used;
    gu.xq = xq;
    gu.xq_stride = xq_stride;
    gu.h = h;
    gu.d_model = D;
    gu.d_ff = F;
    launch_grouped_gate_up<false>(L->qt_gate, KK_GGATE_UP, dim3((unsigned)(F / kGuRows), (unsigned)E), st, gu);
    const size_t hq_rows = P * (size_t)(F / 256);
    hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((hq_rows + 15) / 16)), dim3(kThreads), 0, st, h, (int)P, F,
                       (int)QT_Q8_K, hq, hq_stride, (const int*)nullptr, 1, (const int*)(off + E), 1);
    GroupedDownArgs dn{};
    dn.down = static_cast<const uint8_t*>(L->down);
    dn.expert_stride = row_bytes(L->qt_down, F) * (size_t)D;
    dn.off = off;
    dn.hq = hq;
    dn.hq_stride = hq_stride;
    dn.y = y;
    dn.d_model = D;
    dn.d_ff = F;
    launch_grouped_down<false>(L->qt_down, KK_GDOWN, D, E, st, dn);
    if (join && !ck(hipStreamWaitEvent(st, join, 0), "join the shared expert")) return -1;
    CombineArgs cb{y, pos_of, d_w, shared, d_resid, d_out, n_used, D};
    const bool v4 = D % 4 == 0 && ((reinterpret_cast<uintptr_t>(d_out) | reinterpret_cast<uintptr_t>(d_resid) |
                                    reinterpret_cast<uintptr_t>(shared)) & 15) == 0;
    if (v4)
        hipLaunchKernelGGL(k_combine<4>, dim3((unsigned)((D + 4 * kThreads - 1) / (4 * kThreads)), (unsigned)n_tokens),
                           dim3(kThreads), 0, st, cb);
    else
        hipLaunchKernelGGL(k_combine<1>, dim3((unsigned)((D + kThreads - 1) / kThreads), (unsigned)n_tokens),
                           dim3(kThreads), 0, st, cb);
    return ck(hipGetLastError(), "grouped layer launch") ? 0 : -1;
}

SABAH_API int sabah_moe_prefill_layer(const sabah_moe_layer_desc* layer, const float* d_x, const int32_t* d_ids,
                                      const float* d_w, int n_used, int n_tokens, float* d_out, const float* d_resid,
                                      void* stream) {
    if (check_layer_desc(layer)) return -1;
    if (!d_x || !d_ids || !d_w || !d_out || n_used <= 0 || n_tokens < 0) return fail("invalid MoE layer arguments");
    if (!grouped_shape_ok(layer))
        return fail("grouped MoE layer: needs gate/up of one type and down each IQ3_S, Q4_K or Q6_K, d_model a "
                    "multiple of 512 up to %d, d_ff a multiple of 256 up to %d, n_experts <= 4096 (got types "
                    "%d/%d/%d, d_model=%d d_ff=%d E=%d)",
                    256 * kGuMaxBlocks, 256 * kDownBlocks, layer->qt_gate, layer->qt_up, layer->qt_down,
                    layer->d_model, layer->d_ff, layer->n_experts);
    if ((size_t)n_tokens * n_used > (size_t)1 << 24) return fail("grouped MoE layer: too many (token, slot) pairs");
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (!check_sticky()) return -1;
    if (n_tokens == 0) return 0;
    ++g_layer_calls;
    g_lookups += (unsigned long long)n_tokens * n_used;
    return moe_prefill_on(layer, d_x, d_ids, d_w, n_used, n_tokens, d_out, d_resid, pick_stream(stream));
}

SABAH_API int sabah_moe_route(const float* d_logits, int n_tokens, int n_experts, int n_used, int norm_w,
                              float w_scale, int32_t* d_ids, float* d_w, void* stream) {
    if (!d_logits || !d_ids || !d_w || n_tokens < 0) return fail("invalid route arguments");
    if (n_experts <= 0 || n_experts > kRouteThreads * kRouteMaxPerThread)
        return fail("route: n_experts %d outside [1, %d]", n_experts, kRouteThreads * kRouteMaxPerThread);
    if (n_used <= 0 || n_used > n_experts || n_used > kRouteMaxUsed)
        return fail("route: n_used %d outside [1, min(n_experts, %d)]", n_used, kRouteMaxUsed);
    if (!(w_scale > 0.0f) || w_scale == __builtin_inff()) return fail("route: w_scale must be positive and finite");
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (n_tokens == 0) return 0;
    const RouteArgs a{d_logits, d_ids, d_w, n_experts, n_used, norm_w ? 1 : 0, w_scale};
    const dim3 grid((unsigned)n_tokens), block(kRouteThreads);
    hipStream_t st = pick_stream(stream);
    const int per = (n_experts + kRouteThreads - 1) / kRouteThreads;
    if (per <= 1) hipLaunchKernelGGL(k_route<1>, grid, block, 0, st, a);
    else if (per <= 2) hipLaunchKernelGGL(k_route<2>, grid, block, 0, st, a);
    else if (per <= 4) hipLaunchKernelGGL(k_route<4>, grid, block, 0, st, a);
    else if (per <= 8) hipLaunchKernelGGL(k_route<8>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(k_route<kRouteMaxPerThread>, grid, block, 0, st, a);
    return ck(hipGetLastError(), "route launch") ? 0 : -1;
}

// ===========================================================================
// synthetic weights (benchmark and test data; not part of the drop-in ABI)
// ===========================================================================
// nearest IQ3_S codebook entry of every 4-tuple of 3-bit levels, by squared
// level distance, lowest index on ties
static int ensure_nearest_table() {
    if (g_nearest_dev) return 0;
    std::vector<uint16_t> tab(4096);
    for (int key = 0; key < 4096; ++key) {
        int best = 0, bestd = 1 << 30;
        for (int e = 0; e < 512; ++e) {
            int dist = 0;
            for (int j = 0; j < 4; ++j) {
                const int lv = (key >> (3 * j)) & 7, ge = (kIq3sGridLevels[e] >> (3 * j)) & 7;
                dist += (lv - ge) * (lv - ge);
            }
            if (dist < bestd) {
                bestd = dist;
                best = e;
            }
        }
        tab[key] = (uint16_t)best;
    }
    if (!ck(hipMalloc(reinterpret_cast<void**>(&g_nearest_dev), 4096 * sizeof(uint16_t)), "encoder table")) return -1;
    if (!ck(hipMemcpy(g_nearest_dev, tab.data(), 4096 * sizeof(uint16_t), hipMemcpyHostToDevice), "encoder table upload"))
        return -1;
    return 0;
}

// Fill n_rows rows of k elements of type qt at d_dst with N(0, sigma) weights
// quantised on the device; element i of the tensor is drawn from (seed, i).
SABAH_API int sabah_synth_weights(void* d_dst, int qt, long long n_rows, int k, unsigned long long seed, float sigma,
                                  void* stream) {
    if (!d_dst || n_rows < 0 || !supported_weight_type(qt) || row_bytes(qt, k) == 0)
        return fail("synth: invalid arguments (type %d, k %d)", qt, k);
    if (g_device < 0) return fail("sabah_rt_init has not been called");
    if (n_rows == 0) return 0;
    if (qt != QT_Q8_0 && qt != QT_Q4_K && qt != QT_Q6_K && qt != QT_IQ3_S)
        return fail("synth: no device encoder for type %d (load the bank's bytes instead)", qt);
    if (qt == QT_IQ3_S && ensure_nearest_table()) return -1;
    const long long nb = n_rows * (long long)(k / block_elems(qt));
    const dim3 grid((unsigned)((nb + 255) / 256));
    hipStream_t st = pick_stream(stream);
    uint8_t* d = reinterpret_cast<uint8_t*>(d_dst);
    switch (qt) {
    case QT_Q8_0: hipLaunchKernelGGL(k_synth<QT_Q8_0>, grid, dim3(256), 0, st, d, nb, (uint64_t)seed, sigma, g_nearest_dev); break;
    case QT_Q4_K: hipLaunchKernelGGL(k_synth<QT_Q4_K>, grid, dim3(256), 0, st, d, nb, (uint64_t)seed, sigma, g_nearest_dev); break;
    case QT_Q6_K: hipLaunchKernelGGL(k_synth<QT_Q6_K>, grid, dim3(256), 0, st, d, nb, (uint64_t)seed, sigma, g_nearest_dev); break;
    case QT_IQ3_S: hipLaunchKernelGGL(k_synth<QT_IQ3_S>, grid, dim3(256), 0, st, d, nb, (uint64_t)seed, sigma, g_nearest_dev); break;
    }
    return ck(hipGetLastError(), "synth launch") ? 0 : -1;
}
