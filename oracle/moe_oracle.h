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

/* Router logits[T][NE] = (bias or 0) + x[T][E] . wr[NE][E]^T
 * (matmul.c:13-33 mma_init, 91-131 GEMV, 169-245 tiled path). */
void orc_router(const float *x, const float *wr, const float *bias,
                size_t T, size_t E, size_t NE, float *logits);

/* In-place softmax over n values (nn.c:221-262, tensor.c:479-517). */
void orc_softmax_1d(float *row, size_t n);

/* top_k with the reference's seeding and strict-greater insertion
 * (nn.c:276-308). ids/w are ascending by weight; slot k-1 is the max. */
void orc_top_k(const float *row, size_t n, uint32_t *ids, float *w, size_t k);

/* fp32-activation dot with one quantized row (quant.c:103-155). */
float orc_dot_quant(const float *x, const void *qrow, int wtype, size_t n);

/* out[T][N] = add + x[T][K] . W^T, W = N rows of K columns in blocks; add
 * NULL, [N] (add_len == N) or [T][N] (matmul.c:13-33,285-312) */
void orc_qmat_mul(const float *x, size_t T, const void *q, int wtype, size_t N, size_t K,
		  const float *add, size_t add_len, float *out);

/* Dequantize one row of n elements (quant.c:157-196). */
void orc_dequant_row(const void *qrow, int wtype, float *dst, size_t n);

/* One expert, one token: out[E] = down . (silu(gate . x) * (up . x))
 * (nn.c:449-493 fused_ffn_fn).  h is a caller scratch of EI floats. */
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

#ifdef __cplusplus
}
#endif
#endif
