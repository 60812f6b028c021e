/*
 * sabah_rt - MI355X-native MoE MUL_MAT_ID expert runtime, C ABI.
 *
 * Drop-in for the runtime library that llama.cpp's Sabah bridge dlopen()s
 * (patches/llama.cpp/0001-sabah-native-mul-mat-id.patch:138-175) and that the
 * Python harness binds with ctypes (sabah/runtime/rt.py:53-114).  Plain
 * pointers and sizes only; device pointers are HIP device memory, `stream`
 * is a hipStream_t used as given (NULL is the HIP null stream); entry points
 * without a stream argument run on the library's own stream.
 *
 * Every int-returning entry point returns 0 on success and -1 on failure with
 * a message readable through sabah_rt_last_error().  The library is not
 * re-entrant: calls that overlap on different host threads or streams share
 * its scratch buffers and error buffer (as the reference's does,
 * sabah_rt.cu:3555-3567).
 */
#ifndef SABAH_RT_H
#define SABAH_RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- lifecycle ---------------------------------------------------------- */

/* Select the device, create the library stream and the sticky error word.
 * Replaces sabah_rt_init (sabah_rt.cu:3190-3199). */
int sabah_rt_init(int device);

/* Release everything sabah_rt_init and the calls since made.
 * Replaces sabah_rt_shutdown (sabah_rt.cu:3221-3232). */
int sabah_rt_shutdown(void);

/* Message of the last failed call.  Replaces sabah_rt_last_error (sabah_rt.cu:3041). */
const char *sabah_rt_last_error(void);

/* "sabah_rt abi=v2 sentinel=0 arch=gfx950".  Replaces sabah_rt_build_info
 * (sabah_rt.cu:3839-3843); this library has no sentinel builds. */
const char *sabah_rt_build_info(void);

/* Number of visible HIP devices.  Replaces sabah_rt_device_count (sabah_rt.cu:3234-3238). */
int sabah_rt_device_count(void);

/* ---- the hooked operator -------------------------------------------------- */

/* ggml MUL_MAT_ID on the HBM-resident expert bank:
 *   dst[t][i][0..rows) = W[ids[t][i]] . x[t][i % x_rows]
 * with x quantised to q8 exactly as ggml's CPU path does (q8_0 for Q8_0, IQ4_NL
 * and Q2_0 weights, q8_1 for Q5_1, q8_K for Q4_K / Q5_K / Q6_K / IQ3_S /
 * IQ3_XXS / IQ2_S / IQ4_XS).  Same 21
 * arguments, order and
 * meaning as sabah_rt_mul_mat_id_v2 (sabah_rt.cu:3494-3515; bridge call
 * 0001 patch:193-200):
 *   source        src0->data: a key registered with sabah_rt_register_bank
 *                 (e.g. the host mmap address llama.cpp holds), or a device
 *                 pointer to the GGUF-layout tensor [n_experts][rows][row_stride]
 *   expert_stride src0->nb[2];  row_stride src0->nb[1] (>= row bytes of qt, k)
 *   d_x           src1->data f32; x_id_stride = nb[1], x_rows = ne[1] (1 or n_ids),
 *                 x_token_stride = nb[2]
 *   d_ids         ids->data int32; ids_id_stride = nb[0], ids_token_stride = nb[1]
 *   n_ids, n_tokens  ids->ne[0], ids->ne[1]; n_tokens == 0 is a counted no-op
 *   d_dst         dst->data f32, rows contiguous; dst_id_stride = nb[1],
 *                 dst_token_stride = nb[2]
 *   rows, k, n_experts, qt   src0->ne[1], ne[0], ne[2], ggml_type
 *                 (7 Q5_1, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 18 IQ3_XXS,
 *                 20 IQ4_NL, 21 IQ3_S, 22 IQ2_S, 23 IQ4_XS, 42 Q2_0;
 *                 k % block size == 0)
 *   stream        hipStream_t the kernel is enqueued on (NULL: the null stream)
 *   ids_key       accepted and ignored: ids are read on the device, never
 *                 downloaded, so there is nothing to reuse.  Callers passing
 *                 only 20 arguments (tests/test_mul_mat_id_contract.py:153-154)
 *                 are therefore safe.
 * Results are valid in stream order on return; the call never synchronises.
 * An expert id outside [0, n_experts) cannot be reported by the call that
 * reads it: that slot's outputs become NaN and the next call (or
 * sabah_rt_check_errors) fails with the message.  With the environment
 * variable SABAH_RT_SYNC_IDS=1 the ids are downloaded and checked first,
 * as the reference does (sabah_rt.cu:3672-3675). */
int sabah_rt_mul_mat_id_v2(const void *source, size_t expert_stride, size_t row_stride,
                           const void *d_x, size_t x_id_stride, int x_rows, size_t x_token_stride,
                           const void *d_ids, size_t ids_id_stride, size_t ids_token_stride,
                           int n_ids, int n_tokens,
                           float *d_dst, size_t dst_id_stride, size_t dst_token_stride,
                           int rows, int k, int n_experts, int qt,
                           void *stream, const void *ids_key);

/* Map a caller-side tensor address range [source_key, source_key + bytes) to
 * the device copy of that expert tensor, so MUL_MAT_ID calls that pass the
 * caller's (host) address run on the HBM-resident bank.  Replaces the
 * residency tier's (source pointer, expert) -> slot lookup
 * (sb_mmid_slot, sabah_rt.cu:748-800): with the whole bank in 288 GB of HBM
 * the lookup is an address offset and never misses. */
int sabah_rt_register_bank(const void *source_key, void *d_base, size_t bytes,
                           size_t expert_stride, int n_experts);
int sabah_rt_unregister_bank(const void *source_key);

/* Fails (and clears the sticky word) if a kernel since the last check met an
 * expert id out of range.  No reference counterpart: the reference checks ids
 * on the host before launching (sabah_rt.cu:3672-3675). */
int sabah_rt_check_errors(void);

/* ---- observability -------------------------------------------------------- */

/* Replaces sabah_rt_get_metrics (sabah_rt.cu:3864-3877).  All-resident bank:
 * every (token, slot) lookup is a hit; misses, evictions and bytes_fetched
 * stay 0; resident_bytes = bytes of all registered banks. */
int sabah_rt_get_metrics(unsigned long long *hits, unsigned long long *misses,
                         unsigned long long *evictions, unsigned long long *bytes_fetched,
                         unsigned long long *resident_bytes);

/* Replaces sabah_rt_get_diag (sabah_rt.cu:3849-3862); overflow and the
 * byte-verification counters have no meaning without a copy tier and stay 0. */
int sabah_rt_get_diag(unsigned long long *calls, unsigned long long *tokens,
                      unsigned long long *overflow, unsigned long long *verify_ok,
                      unsigned long long *verify_fail);

/* Counters as one JSON object.  Replaces sabah_rt_snapshot (sabah_rt.cu:3835-3837). */
int sabah_rt_snapshot(char *buf, size_t n);

/* ---- harness entry points ----------------------------------------------- */

/* Device memory, pinned host memory, copies, events and the two library
 * streams, for the Python harness: the reference's rt.lib() binds these by
 * name (sabah/runtime/rt.py:70-107) and its executor, expert bank and hot
 * tier call them.  Same names, signatures and return conventions as
 * sabah_rt.cu:3240-3353: allocators return NULL on failure (message in
 * sabah_rt_last_error); int calls return 0 / -1; sabah_event_query returns
 * 1 (complete), 0 (in flight) or -1; sabah_event_elapsed_ms waits for b and
 * returns -1 on error.  The copy stream is the library's second stream
 * (sabah_h2d_async, sabah_event_record_copy, sabah_copy_wait_event); the
 * compute stream is the one sabah_moe_block and sabah_dequant use.
 * sabah_host_alloc returns pinned memory from hipHostMalloc (the reference
 * pools and reuses its pinned blocks; here each call allocates). */
void *sabah_dev_alloc(size_t bytes);
void sabah_dev_free(void *p);
void *sabah_host_alloc(size_t bytes);
void sabah_host_free(void *p);
int sabah_dev_mem(size_t *free_bytes, size_t *total_bytes);
int sabah_memcpy_h2d(void *dst, const void *src, size_t n);
int sabah_memcpy_d2h(void *dst, const void *src, size_t n);
int sabah_memset_d(void *dst, int v, size_t n);
int sabah_h2d_async(void *dst, const void *src, size_t n);
void *sabah_event_create(void);
void sabah_event_destroy(void *ev);
int sabah_event_record_copy(void *ev);
int sabah_event_record_compute(void *ev);
int sabah_compute_wait_event(void *ev);
int sabah_copy_wait_event(void *ev);
float sabah_event_elapsed_ms(void *a, void *b);
int sabah_event_sync(void *ev);
int sabah_event_query(void *ev);
int sabah_sync_copy(void);
int sabah_sync_compute(void);
int sabah_sync_all(void);

/* A device slab: one allocation of capacity_bytes whose ranges are handed
 * out (256-byte aligned) and returned.  Replaces sabah_slab_* (sabah_rt.cu:
 * 3889-3903, allocator 332-420), which backs the reference's VRAM tier; the
 * HBM-resident bank needs no tier, and the slab remains for harness callers.
 * init on an existing slab is a no-op; alloc returns NULL when no free range
 * fits; free merges the range with its free neighbours. */
int sabah_slab_init(size_t capacity_bytes);
void *sabah_slab_alloc(size_t bytes);
void sabah_slab_free(void *ptr);
void sabah_slab_destroy(void);

/* n elements of type qt (a whole number of blocks) at host address src,
 * decoded into n floats at host address dst.  Replaces sabah_rt_host_dequant
 * (sabah_rt.cu:3845-3847), whose decoders run on the host; here the bytes are
 * decoded on the device by the same decoders as sabah_dequant.  Synchronous;
 * callable before sabah_rt_init, like the reference's (the library is then
 * initialised on the current HIP device).  Returns -1 for an unsupported type
 * or a partial block. */
int sabah_rt_host_dequant(const void *src, float *dst, int qt, int n);

/* Bytes of one row of n elements of type qt (0 if unsupported or n is not a
 * whole number of blocks).  Replaces sabah_row_bytes (sabah_rt.cu:3887). */
size_t sabah_row_bytes(int qt, int n);

/* Dequantise n_rows rows of row_elems elements, device to device, through the
 * same item decoders the dot kernels use, in ggml dequantize_row_* float
 * order; synchronises the library stream.  Replaces sabah_dequant
 * (sabah_rt.cu:3879-3885, kernel k_dequant 3016-3034). */
int sabah_dequant(const void *d_src, float *d_dst, int qt, int n_rows, int row_elems);

/* Quantise n_rows rows of k floats (device) into ggml's activation block
 * layout for weight type qt (block_q8_0 or block_q8_K), device to device,
 * on `stream`.  No reference counterpart: the reference feeds its kernels
 * fp32 activations; this exposes the q8 step for byte-level checks. */
int sabah_quantize_act(const float *d_x, void *d_y, int qt, int n_rows, int k, void *stream);

/* One routed-MoE block for one token on the library stream, with a device
 * pointer table [gate x n_used, up x n_used, down x n_used] and router weights:
 *   d_out (+)= sum_k w_k * down_k( silu(gate_k . x) * (up_k . x) )
 * d_h receives the n_used x ff SwiGLU rows.  Same signature and pointer layout
 * as sabah_moe_block (sabah_rt.cu:3356-3378). */
int sabah_moe_block(const float *d_x, float *d_out, float *d_h, const void *const *d_ptrs,
                    const float *d_w, int d_model, int ff, int n_used,
                    int qt_gate, int qt_up, int qt_down, int accumulate);

/* A MoE layer over n_tokens tokens with ids read on the device from the bank
 * bases (no pointer table), plus an optional dense shared expert (optionally
 * sigmoid-gated) and an optional residual.  Generalises sabah_moe_block
 * (sabah_rt.cu:3362-3378) to the ggml graph's batched form (qwen4exp.cpp:848-892):
 *   out[t] = [resid[t] +] sum_k w[t][k] * y[t][k] [+ g[t] * shared(x[t])]
 * with g[t] = sigmoid(shared_gate_inp . x[t]), or 1 without a gate row.
 * Bank bases are device memory in GGUF layout [n_experts][rows][row_bytes]. */
typedef struct sabah_moe_layer_desc {
    const void *gate, *up, *down;
    int qt_gate, qt_up, qt_down;
    int d_model, d_ff, n_experts;
    const void *shared_gate, *shared_up, *shared_down;   /* NULL: no shared expert */
    int qt_shared_gate, qt_shared_up, qt_shared_down;
    int d_ff_shared;
    /* Optional f32 [d_model] row (ffn_gate_inp_shexp): the shared expert's
     * output for token t is multiplied by sigmoid(shared_gate_inp . x[t])
     * before it is added (qwen4exp.cpp:877-885).  NULL adds it unscaled. */
    const float *shared_gate_inp;
} sabah_moe_layer_desc;

int sabah_moe_layer(const sabah_moe_layer_desc *layer, const float *d_x, const int32_t *d_ids,
                    const float *d_w, int n_used, int n_tokens, float *d_out, const float *d_resid,
                    void *stream);

/* sabah_moe_layer with the same arguments and bit-identical results, for
 * callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  No reference
 * counterpart (the reference allocates its staging at init and on growth).
 * Every piece of device scratch the layer needs (h, the shared expert's
 * rows, q8 rows of h) comes from one static device array of 8 MiB that the
 * library holds on each GPU until the process ends; the call allocates
 * nothing and never synchronises.  A call whose scratch exceeds 8 MiB
 * (about 200 tokens x top-10 at d_ff 768) fails before enqueuing anything.
 * Calls on one GPU share the array: calls that overlap on different streams
 * race.  Kernel timing does not record its launches. */
int sabah_moe_layer_noalloc(const sabah_moe_layer_desc *layer, const float *d_x, const int32_t *d_ids,
                            const float *d_w, int n_used, int n_tokens, float *d_out, const float *d_resid,
                            void *stream);

/* n_layers MoE layers in sequence on a residual stream:
 *   x <- x + layer_l(x)  for l = 0 .. n_layers-1
 * with per-layer ids/weights at d_ids + l*n_tokens*n_used (same for d_w).
 * d_x is updated in place.  No reference counterpart: it is the decode
 * workload the reference's per-call path serves 48 times per token
 * (REPORT.md:283-290), issued as one call. */
int sabah_moe_chain(const sabah_moe_layer_desc *layers, int n_layers, float *d_x,
                    const int32_t *d_ids, const float *d_w, int n_used, int n_tokens, void *stream);

/* The same layer as sabah_moe_layer (same arguments, bit-identical results),
 * computed group-major for a batch of tokens (prefill): the (token, slot)
 * pairs are grouped by expert on the device, and each routed expert's rows
 * are read once and applied to all of its pairs with int8 MFMA.  No
 * reference counterpart: the reference's kernel re-reads an expert per
 * (token, slot) (sabah_rt.cu:2791-2839); the grouping follows upstream
 * ggml's sorted MUL_MAT_ID fallback (ggml-cuda.cu:1985-2082).  Needs gate and
 * up of one type and down of any, each IQ3_S, Q4_K or Q6_K, d_model a multiple
 * of 512 up to 2048, d_ff a multiple of 256 up to 1024, n_experts <= 4096;
 * returns -1 otherwise.  An out-of-range id
 * makes its token's output NaN and fails the next call, as in sabah_moe_layer. */
int sabah_moe_prefill_layer(const sabah_moe_layer_desc *layer, const float *d_x, const int32_t *d_ids,
                            const float *d_w, int n_used, int n_tokens, float *d_out, const float *d_resid,
                            void *stream);

/* Router gating for n_tokens rows of n_experts router logits (device f32),
 * as ggml's graph runs it before MUL_MAT_ID (qwen4exp.cpp:848-862 ->
 * build_moe_ffn with softmax gating; upstream's fused topk-moe,
 * ggml-cuda.cu:3390-3405):
 *   p = softmax(logits[t])                       (ggml_soft_max; exp sums in double)
 *   d_ids[t] = the n_used largest p, descending  (ggml_argsort_top_k; ties: lower index first)
 *   d_w[t] = p[d_ids[t]], divided by their sum when norm_w (ggml_sum_rows, ggml_div),
 *            times w_scale when w_scale != 1 (ggml_scale)
 * so the fused layer's ids and weights never leave the device.  No reference
 * counterpart: the reference's runtime receives ids from ggml.  n_experts <=
 * 4096, n_used <= min(n_experts, 64), w_scale > 0; enqueued on `stream`. */
int sabah_moe_route(const float *d_logits, int n_tokens, int n_experts, int n_used, int norm_w,
                    float w_scale, int32_t *d_ids, float *d_w, void *stream);

/* How sabah_rt_mul_mat_id_v2 runs IQ3_S, Q4_K and Q6_K calls over many tokens.  No reference
 * counterpart: the reference's kernel re-reads an expert per (token, slot)
 * (sabah_rt.cu:2791-2839).  Grouped, the (token, slot) pairs are grouped by
 * expert on the device and each expert is read once per call (int8 MFMA);
 * eligible calls have packed rows, dense ids and x, n_experts <= 4096, and
 * k <= 1024 with rows % 64 == 0, or k % 512 == 0, k <= 2048, rows % 32 == 0.
 * mode 0 (default): grouped when eligible with at least 1 (IQ3_S with
 * k <= 1024, and Q6_K) or 2 (otherwise) pairs per expert on average; 1: never;
 * 2: whenever eligible.
 * The results are bit-identical either way.  Grouped calls use library
 * scratch (pair lists, q8 rows) shared by every stream: calls that may
 * overlap on different streams need mode 1 (the token-major kernel uses no
 * scratch).  Returns -1 for another mode. */
int sabah_rt_set_mmid_grouping(int mode);

#ifdef __cplusplus
}
#endif

#endif /* SABAH_RT_H */
