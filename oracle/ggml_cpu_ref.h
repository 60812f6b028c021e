/*
 * ORACLE - test infrastructure only.
 *
 * A plain-C restatement of ggml's CPU MUL_MAT_ID path for the eight expert
 * formats (Q8_0, Q5_1, Q4_K, Q5_K, Q6_K, IQ3_S, IQ3_XXS, IQ2_S, IQ4_NL, IQ4_XS,
 * Q2_0), used as
 * the checker for the HIP kernels.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library never links or calls it.
 *
 * ggml itself (llama.cpp @ 96ffdc41ceb055e1c2d3d96667ae6d9f0ccb710b, pinned in
 * third_party/llama.cpp.version:1-2) is not vendored in the reference, so the
 * algorithm is restated from its published form and anchored on the
 * reference's own call sites and format readers; each function below cites
 * them.
 *
 * How each function is pinned (tests/test_oracle_formats.py,
 * tests/test_oracle_tables.py, tests/test_golden_trace.py):
 *   orc_fp16_to_fp32 / orc_fp32_to_fp16: every finite half; numpy's
 *     round-to-nearest-even conversion on random values and exact ties.
 *   orc_quantize_q8_0: hand-computed blocks; halves rounded away from zero
 *     (quants.py:413-427, np_roundf 44-48); the all-zero block.
 *   orc_quantize_q8_1: the q8_0 bytes (same d and q) plus s = fp16(d * sum q),
 *     hand-computed blocks and the all-zero block.
 *   orc_quantize_q8_K: hand-computed blocks; ties to even; the scale takes
 *     the sign of the first maximum; clamp at 127; zero block; bsums
 *     (tools/rc4/opcheck.py:73-80).
 *   Q5_1 / Q5_K dequantisation: known-answer blocks (the fifth bit of
 *     element i is bit i of qh for Q5_1, bit j of qh[l] for element l of
 *     Q5_K sub-block j; d, m / dmin, 6-bit scales and mins) from
 *     sabah_rt.cu:2241-2290 and quants.py:367-409, 559-583; Q5_K equals Q4_K
 *     on the same scale and nibble bytes when qh is zero.
 *   orc_dequantize_row: known-answer blocks per format (d = 1, unit scales,
 *     codebook rows, sign / qh / scale bits) from the closed forms of
 *     sabah_rt.cu:2233-2423 and quants.py:412-435, 509-556, 586-606, 1091-1159.
 *   the IQ3_S codebook: equal to both reference copies (sabah_iq_tables.h:
 *     638-704 and quants.py:1094-1127 grid_hex) and to its recorded sha256.
 *   the IQ3_XXS and IQ2_S codebooks, the IQ2_XXS/IQ3_XXS sign bytes and the IQ4 levels:
 *     generated from quants.py text (oracle/gen_iq_tables.py), equal to the
 *     reference's second copy (sabah_iq_tables.h) and to recorded sha256
 *     values; closed forms (ksigns = index with an even-parity bit 7, levels
 *     sorted, grid bytes among the eight magnitudes).
 *   IQ3_XXS / IQ2_S / IQ4_NL / IQ4_XS dequantisation: known-answer blocks
 *     (grid row, sign bytes, 4-bit scale; grid index high bits from qh and
 *     the two scale nibbles; level bytes and d; 6-bit sub-block scales) from
 *     sabah_rt.cu:2293-2344, 2380-2409 and quants.py:935-1075, 1364-1411.
 *   orc_vec_dot: the float64 dot of the decoded operands (all formats; for
 *     Q5_1 the q8_1 s term equals d_x times the block's q sum); the
 *     IQ3_S integer block sums exactly; IQ3_XXS exactly a quarter and IQ2_S
 *     exactly an eighth of their integer sums; the Q4_K min term through
 *     bsums.
 *   orc_mul_mat_id / orc_moe_layer: brute-force loops; bad ids and geometry
 *     rejected; a layer is the composition of its MUL_MAT_IDs; the shared
 *     expert is added last; duplicate ids of the reference's recorded routing
 *     trace give identical slot outputs.
 *   orc_quantize_weights: round trip (its output only has to be valid input).
 * Parity unpinned: the fp32 accumulation order inside orc_vec_dot for Q4_K,
 * Q5_K and Q6_K (ggml's generic eight-lane order, restated from its published
 * source, which cannot be built or run here).  Checks against those three use
 * the floating-point tolerance, not bit equality.  The other formats sum one
 * fp32 term per block (per 32-element sub-block for IQ4_XS) serially in block
 * order, the HIP kernels do the same, and their outputs are compared bit for
 * bit.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type codes (sabah/runtime/rt.py:20-23 uses the same enum values). */
enum {
    ORC_F32 = 0,
    ORC_Q5_1 = 7,
    ORC_Q8_0 = 8,
    ORC_Q8_1 = 9,
    ORC_Q4_K = 12,
    ORC_Q5_K = 13,
    ORC_Q6_K = 14,
    ORC_Q8_K = 15,
    ORC_IQ3_XXS = 18,
    ORC_IQ2_S = 22,
    ORC_IQ4_NL = 20,
    ORC_IQ3_S = 21,
    ORC_IQ4_XS = 23,
    ORC_Q2_0 = 42,
};

/* Block geometry: elements and bytes per block (sabah_rt.cu:2155-2184;
 * Q6_K from quants.py:586-606 and model_inspector.py:34). */
int orc_block_elems(int qt);
int orc_block_bytes(int qt);
size_t orc_row_bytes(int qt, int n);
/* the activation format ggml's CPU quantises src1 into for weight type qt */
int orc_vec_dot_type(int qt);

/* IEEE binary16 conversion; fp32 -> fp16 rounds to nearest even. */
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);

/* Activation quantisers (ggml quantize_row_q8_0_ref / quantize_row_q8_1_ref /
 * quantize_row_q8_K_ref). */
void orc_quantize_q8_0(const float *x, uint8_t *y, int k);
void orc_quantize_q8_1(const float *x, uint8_t *y, int k);
void orc_quantize_q8_K(const float *x, uint8_t *y, int k);
/* quantise a row of k floats into the activation format for weight type qt */
int orc_quantize_act(int qt, const float *x, uint8_t *y, int k);
size_t orc_act_row_bytes(int qt, int k);

/* Weight encoders.  Q8_0 follows ggml's reference quantiser; Q4_K, Q6_K and
 * IQ3_S are simple valid encoders of this project's own (parity is judged on
 * decoding the same bytes, not on encoder quality). */
int orc_quantize_weights(int qt, const float *x, uint8_t *y, int k);

/* Decode a row of k elements (ggml dequantize_row_*). */
int orc_dequantize_row(int qt, const uint8_t *x, float *y, int k);

/* One dot product of a weight row with a quantised activation row
 * (ggml_vec_dot_{q8_0_q8_0, q4_K_q8_K, q6_K_q8_K, iq3_s_q8_K}). */
float orc_vec_dot(int qt, const uint8_t *w, const uint8_t *a, int k);

/* MUL_MAT_ID on host buffers with the sabah_rt_mul_mat_id_v2 argument
 * meaning (sabah_rt.cu:3494-3515): dst[t][i][r] = W[ids[t][i]][r] . q8(x[t][i % x_rows]).
 * Returns 0, or -1 on invalid arguments.  n_threads <= 0 means all cores. */
int orc_mul_mat_id(const void *source, size_t expert_stride, size_t row_stride,
                   const float *x, size_t x_id_stride, int x_rows, size_t x_token_stride,
                   const int32_t *ids, size_t ids_id_stride, size_t ids_token_stride,
                   int n_ids, int n_tokens,
                   float *dst, size_t dst_id_stride, size_t dst_token_stride,
                   int rows, int k, int n_experts, int qt, int n_threads);

/* The gated expert FFN of one MoE layer as ggml's graph runs it
 * (qwen4exp.cpp:848-862 -> build_moe_ffn; executor.py:1-16):
 *   g = MUL_MAT_ID(gate), u = MUL_MAT_ID(up), h = silu(g) * u,
 *   y = MUL_MAT_ID(down, h), out = sum_k (y_k * w_k)   (serial over k)
 * plus, when shared_gate != NULL, a dense shared expert added last:
 *   out += g * down_s(silu(gate_s x) * up_s x)
 * with g = sigmoid(shared_gate_inp . x) when shared_gate_inp != NULL
 * (qwen4exp.cpp:877-885: ggml_mul_mat, ggml_sigmoid, ggml_mul, ggml_add),
 * else 1 (no multiply).  The gate's dot product is summed in double. 
 * Expert tensors are [n_experts][rows][row_bytes] (GGUF layout).
 * x [n_tokens][d_model], ids/w [n_tokens][n_used], out [n_tokens][d_model]. */
typedef struct {
    const void *gate, *up, *down;
    int qt_gate, qt_up, qt_down;
    int d_model, d_ff, n_experts;
    const void *shared_gate, *shared_up, *shared_down;   /* optional */
    int qt_shared_gate, qt_shared_up, qt_shared_down;
    int d_ff_shared;
    const float *shared_gate_inp;                         /* optional [d_model] */
} orc_moe_layer_desc;

int orc_moe_layer(const orc_moe_layer_desc *L, const float *x, const int32_t *ids,
                  const float *w, int n_used, int n_tokens, float *out,
                  float *h_out /* optional [n_tokens][n_used][d_ff] */, int n_threads);

/* Router gating as ggml's CPU ops run it (qwen4exp.cpp:848-862 ->
 * build_moe_ffn, softmax gating):
 *   soft_max: m = max_i l_i (in order), e_i = expf(l_i - m), S = sum_i e_i in
 *             double (in order), p_i = e_i * (float)(1.0 / S)
 *   argsort_top_k: the n_used largest p, descending; ties to the lower index
 *   get_rows, then with norm_w sum_rows (double, in order) and div; then
 *   times w_scale when w_scale != 1 (ggml_scale).
 * logits [n_tokens][n_experts], ids / w [n_tokens][n_used]. */
int orc_moe_route(const float *logits, int n_tokens, int n_experts, int n_used, int norm_w, float w_scale,
                  int32_t *ids, float *w);

#ifdef __cplusplus
}
#endif
