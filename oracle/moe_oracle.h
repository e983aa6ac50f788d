/*
 * CPU oracle for the quantized mixture-of-experts FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the
 * reference's CPU algorithm (hoathienvu8x/llm.c, AVX2 build) used as the
 * checker for the HIP kernels.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links
 * or calls it.
 *
 * Every function reproduces the reference's floating-point operation order
 * for an AVX2 build (8 fp32 lanes, fused multiply-add, the fixed horizontal
 * reduction tree of vector_avx2.h:126-132, glibc expf, IEEE division), so
 * router logits, expert ids and routing weights are bit-identical to the
 * reference.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* values of the reference's enum tensor_dtype (tensor.h:10-17) */
#define ORC_Q8_0 1
#define ORC_Q4_0 2
#define ORC_Q4_K 3
#define ORC_Q6_K 5

/* Router logits[T][NE] = (bias or 0) + x[T][E] . wr[NE][E]^T
 * (matmul.c:13-33 mma_init, 91-131 GEMV, 169-245 tiled path). */
void orc_router(const float *x, const float *wr, const float *bias,
                size_t T, size_t E, size_t NE, float *logits);

/* dot_f32_f32 (matmul.c:91-105): 8 FMA lane chains, the lane tree, an FMA
 * scalar tail. */
float orc_dot_f32(const float *x, const float *y, size_t n);

/* In-place softmax over n values (nn.c:221-262, tensor.c:479-517). */
void orc_softmax_1d(float *row, size_t n);

/* top_k with the reference's seeding and strict-greater insertion
 * (nn.c:276-308). ids/w are ascending by weight; slot k-1 is the max. */
void orc_top_k(const float *row, size_t n, uint32_t *ids, float *w, size_t k);

/* fp32-activation dot with one quantized row (quant.c:103-155, 198-418;
 * dot_f32_quant, quant.c:577-614). */
float orc_dot_quant(const float *x, const void *qrow, int wtype, size_t n);

/* out[T][N] = add + x[T][K] . W^T, W = N rows of K columns in blocks; add
 * NULL, [N] (add_len == N) or [T][N] (matmul.c:13-33,285-312); K-quant
 * matrices with K % 256 == 0 take the Q8_K path of the -DQ8_DOT build */
void orc_qmat_mul(const float *x, size_t T, const void *q, int wtype, size_t N, size_t K,
		  const float *add, size_t add_len, float *out);

/* Dequantize one row of n elements (quant.c:157-196, 420-531). */
void orc_dequant_row(const void *qrow, int wtype, float *dst, size_t n);

/* quantize_row_q8 (quant.c:627-654): n/256 Q8_K blocks as d[n/256],
 * qs[n], bsums[n/256][16]. */
void orc_quantize_q8k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums);

/* dot_q4_K_q8_K / dot_q6_K_q8_K (quant_cpu.h:7-120 = quant_avx2.h:8-209) of
 * one Q4_K/Q6_K row of n values with Q8_K activations. */
float orc_dot_q8k(const float *yd, const int8_t *q8, const int16_t *bsums, const void *qrow,
                  int wtype, size_t n);

/* One expert, one token: out[E] = down . (silu(gate . x) * (up . x))
 * (nn.c:449-493 fused_ffn_fn).  h is a caller scratch of EI floats.
 * wtype: the gate/up block type, or'ed with the down type << 8 where that
 * differs (a Q4_K_M file's Q4_K gate/up with Q6_K down: 3 | 5 << 8); the
 * same encoding runs through orc_moe_ffn and the model oracles. */
void orc_fused_ffn(const float *x, const void *gate, const void *up,
                   const void *down, int wtype, size_t E, size_t EI,
                   float *h, float *out);

/* Whole MoE FFN layer (olmoe.c:343-407; llama.c:393-457 when renorm != 0).
 * gate_e/up_e/down_e are per-expert base pointers to row-major blocks.
 * ids_out/w_out/logits_out/probs_out are optional ([T][topk], [T][NE]).
 * Tokens are independent, so nthreads > 1 splits them over threads without
 * changing any result bit. */
void orc_moe_ffn(const float *x, float *out, size_t T,
                 const float *wr, const float *bias,
                 const void *const *gate_e, const void *const *up_e,
                 const void *const *down_e, int wtype,
                 size_t E, size_t EI, size_t NE, size_t topk, int renorm,
                 uint32_t *ids_out, float *w_out, float *logits_out,
                 float *probs_out, int nthreads);

/* glibc expf over an array (the function vector_avx2.h:50-63 calls). */
void orc_expf_array(const float *in, float *out, size_t n);

/* glibc expf of every float whose bit pattern lies in [bits0, bits0+n). */
void orc_expf_bits(uint32_t bits0, size_t n, float *out, int nthreads);

/*
 * The reference's threading for timing the oracle as the CPU baseline: a
 * persistent pool of nthreads spinning workers (the calling thread is one
 * of them); each operation then runs on one thread below 16 Mi flops and
 * on all of them above (thread_pool.c:25,178-185,208-238).  nthreads <= 1
 * turns it off (the default: operations run on the calling thread; the
 * nthreads arguments below split tokens instead).  Results do not change.
 * Returns the pool size, 0 when off, -1 on failure.
 */
int orc_set_pool(int nthreads);

/*
 * The OLMoE model (models/olmoe/olmoe.c) in decode mode, one token per
 * call: embedding (tensor_pick_rows tensor.c:263-294), per layer RMSNorm
 * (nn.c:8-51), q/k/v products, full-vector q/k RMSNorm, RoPE (nn.c:192-219),
 * attention over the fp32 KV cache (olmoe.c:214-341, kvcache.c), output
 * product and residual, RMSNorm, moe_ffn (olmoe.c:343-407), residual; the
 * final RMSNorm and the lm_head product (olmoe.c:497-501,558-564).
 * ptrs: 3 + 12 * layers pointers, token_embd, output, output_norm, then per
 * layer attn_norm, attn_q, attn_k, attn_v, attn_q_norm, attn_k_norm,
 * attn_output, ffn_norm, ffn_gate_inp, ffn_gate_exps, ffn_up_exps,
 * ffn_down_exps (quantized in wtype blocks; norms and router fp32).
 */
typedef struct orc_olmoe orc_olmoe;

orc_olmoe *orc_olmoe_new(size_t layers, size_t E, size_t H, size_t V, size_t NE, size_t topk,
                         size_t EI, size_t C, float theta, int wtype, const void *const *ptrs);
/* the same with a block type per quantized tensor, as a GGUF's tensors carry
 * them: types[0] token_embd, types[1] output, then per layer attn_q, attn_k,
 * attn_v, attn_output, ffn_gate/up_exps, ffn_down_exps (2 + 6 * layers) */
orc_olmoe *orc_olmoe_new_typed(size_t layers, size_t E, size_t H, size_t V, size_t NE,
                               size_t topk, size_t EI, size_t C, float theta, const int *types,
                               const void *const *ptrs);

/* olmoe_decode (olmoe.c:509-520) of token tok at position pos, then the
 * lm_head product into logits[V] (optional).  Optional traces per layer:
 * moe_in [layers][E] (the router's input), ids/w [layers][topk].
 * Returns the greedy pick (main.c:189-193: first maximum). */
int orc_olmoe_decode(orc_olmoe *m, int tok, int pos, float *logits, float *trace_moe_in,
                     uint32_t *trace_ids, float *trace_w, int nthreads);

/* The prompt token by token, then n_gen greedy steps (the model's own
 * position counter advances): tokens[0..n_gen], logits [n_gen+1][V]. */
void orc_olmoe_run(orc_olmoe *m, const int *prompt, size_t n_prompt, size_t n_gen,
                   float *logits, int *tokens, int nthreads);

void orc_olmoe_free(orc_olmoe *m);

/*
 * The Mixtral model (models/llama/llama.c with experts) in decode mode:
 * as the OLMoE model without q/k norms, with QH query and KVH kv heads of
 * E / QH (grouped-query attention), the FLASH_ATTENTION build's
 * flash_attention (nn.c:544-655) with an optional sliding window, and
 * renormalised top-k routing (llama.c:422-427).  ptrs: 3 + layers * (7 + 3
 * * NE) pointers, token_embd, output, output_norm, then per layer
 * attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate_inp,
 * the NE gate, NE up and NE down expert matrices.
 */
typedef struct orc_llama orc_llama;

orc_llama *orc_llama_new(size_t layers, size_t E, size_t QH, size_t KVH, size_t V, size_t NE,
                         size_t topk, size_t EI, size_t C, float theta, size_t window,
                         int wtype, const void *const *ptrs);
orc_llama *orc_llama_new_typed(size_t layers, size_t E, size_t QH, size_t KVH, size_t V,
                               size_t NE, size_t topk, size_t EI, size_t C, float theta,
                               size_t window, const int *types, const void *const *ptrs);
int orc_llama_decode(orc_llama *m, int tok, int pos, float *logits, float *trace_moe_in,
                     uint32_t *trace_ids, float *trace_w, int nthreads);
void orc_llama_run(orc_llama *m, const int *prompt, size_t n_prompt, size_t n_gen,
                   float *logits, int *tokens, int nthreads);
void orc_llama_free(orc_llama *m);

#ifdef __cplusplus
}
#endif
#endif
