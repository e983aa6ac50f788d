/*
 * moe_synth.h - seeded synthetic MoE layer inputs in GGUF block layout.
 *
 * The reference ships no offline MoE weights (its fixtures are downloaded
 * GGUFs), so benchmarks and tests generate layers of the real shapes:
 * N(mean, std) values from a counter-based generator (splitmix64 finaliser as
 * the hash, Box-Muller in double), quantized with the reference's own
 * quantizers:
 *   Q8_0: quantize_row_q8_0  (quant.c:62-78; fp16 scale rounded to nearest
 *         even as F16C _cvtss_sh does, quant.c:46-60)
 *   Q4_0: quantize_q4_0_block (test/quant.c:45-79; truncating fp16 scale,
 *         nibble = clamp(roundf(x*7/amax) + 8, 0, 15))
 *   Q4_K, Q6_K: min/max quantizers into the reference's block formats
 *         (quant.h:30-57; the reference itself only reads such blocks)
 * Element i of stream s under seed k is a pure function of (k, s, i), so
 * generation can be split over threads without changing a bit.
 */
#ifndef MOE_SYNTH_H
#define MOE_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of one row of n elements in block type wtype (1 = Q8_0, 2 = Q4_0,
 * 3 = Q4_K, 5 = Q6_K). */
size_t moe_row_bytes(int wtype, size_t n);

/* out[i] = (float)(mean + std * N_i), i in [0, n), N_i ~ N(0,1). */
void moe_synth_normal(uint64_t seed, uint64_t stream, float mean, float std,
                      float *out, size_t n, int nthreads);

/* quant.c:62-78 */
void moe_quantize_q8_0(const float *x, void *blocks, size_t n);
/* test/quant.c:45-79 */
void moe_quantize_q4_0(const float *x, void *blocks, size_t n);
/* K-quant block formats (quant.h:30-57) by min/max quantizers of this
 * library's own: Q4_K per-32 scale and min, Q6_K signed per-16 scales. */
void moe_quantize_q4_K(const float *x, void *blocks, size_t n);
void moe_quantize_q6_K(const float *x, void *blocks, size_t n);

/* rows x cols matrix of N(0, std) values, quantized row by row into
 * rows * moe_row_bytes(wtype, cols) bytes at blocks. */
void moe_synth_quant_matrix(uint64_t seed, uint64_t stream, float std,
                            int wtype, size_t rows, size_t cols, void *blocks,
                            int nthreads);

/* Stream ids used for one layer's tensors (layer l, expert e). */
uint64_t moe_stream_router(uint64_t layer);
uint64_t moe_stream_bias(uint64_t layer);
uint64_t moe_stream_gate(uint64_t layer, uint64_t expert);
uint64_t moe_stream_up(uint64_t layer, uint64_t expert);
uint64_t moe_stream_down(uint64_t layer, uint64_t expert);
uint64_t moe_stream_input(uint64_t call);
/* The model tensors around the MoE layers: layer l's tensor of kind k
 * (MOE_T_*); tensors outside the layers use layer MOE_T_GLOBAL. */
uint64_t moe_stream_tensor(uint64_t layer, uint64_t kind);
#define MOE_T_ATTN_Q 0
#define MOE_T_ATTN_K 1
#define MOE_T_ATTN_V 2
#define MOE_T_ATTN_O 3
#define MOE_T_ATTN_NORM 4
#define MOE_T_Q_NORM 5
#define MOE_T_K_NORM 6
#define MOE_T_FFN_NORM 7
#define MOE_T_TOKEN_EMBD 8
#define MOE_T_OUTPUT 9
#define MOE_T_OUTPUT_NORM 10
#define MOE_T_PROMPT 11
#define MOE_T_GLOBAL 0xffffffffu

/* f32 -> f16 round-to-nearest-even (as F16C _cvtss_sh(x, 0)) and the exact
 * f16 -> f32, exposed for tests. */
uint16_t moe_f32_to_f16_rne(float f);
float moe_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
