/*
 * hip_moe.h - C ABI of the MI355X (gfx950) quantized mixture-of-experts FFN.
 *
 * Drop-in for the body of the reference's moe_ffn:
 *   models/olmoe/olmoe.c:343-407   (OLMoE: softmax top-k, no renormalisation)
 *   models/llama/llama.c:393-457   (Mixtral: top-k weights renormalised)
 * and everything below it on that call (router GEMV/GEMM matmul.c:270-324,
 * softmax_1d nn.c:221-262, top_k nn.c:276-308, fused_ffn_silu nn.c:496-539,
 * the Q8_0/Q4_0 dots quant.c:103-155, the combine tensor.c:334-353,435-456).
 *
 * Plain C: pointers, sizes and ints only.  Conventions follow the
 * reference's fused_ffn_silu (nn.h:33-39): an int return of 1 means "done",
 * 0 means "not applicable" (unsupported type or shape, no device, HIP error),
 * in which case the caller runs its own CPU body.  Errors are also printed to
 * stderr and kept for hip_moe_last_error().  Nothing here calls exit().
 *
 * Expert ids and routing weights are bit-identical to the reference's AVX2
 * build on every path; layer outputs agree with it to ~1e-6 relative L2 on
 * the fp32 paths (decode, GEMV) and ~5e-4 on the grouped f16-MFMA path taken
 * for many tokens per expert (bound: 1e-3).  See HIP_MOE_PATH_* below.
 *
 * Threading: a layer object owns device scratch; calls on the same layer
 * object must not overlap (the reference is single-threaded per model too,
 * thread_pool.c:45).  Calls that pass no stream share one library stream per
 * device.
 */
#ifndef HIP_MOE_H
#define HIP_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight block types: the reference's enum tensor_dtype values (tensor.h:10-17).
 * Q8_0 = 34-byte blocks {f16 d; int8 qs[32]}, Q4_0 = 18-byte blocks
 * {f16 d; uint8 qs[16]} (quant.h:14-26), rows of cols/32 blocks, row-major. */
#define HIP_MOE_Q8_0 1
#define HIP_MOE_Q4_0 2
#define HIP_MOE_Q4_K 3 /* hip_moe_upload_typed and hip_moe_qmat_* */
#define HIP_MOE_Q6_K 5 /* hip_moe_upload_typed and hip_moe_qmat_* */

typedef struct hip_moe_layer hip_moe_layer;

/*
 * Upload one MoE layer's weights to device memory, once, as GGUF blocks that
 * keep their bytes (gate/up rows as they are, plus a second gate/up copy in
 * 32-row groups for the grouped GEMMs; down matrices regrouped into panels
 * of one block per row).  Replaces the residency of
 *   olmoe_load  (olmoe.c:179-182: ffn_gate_inp + stacked *_exps tensors) and
 *   llama_load  (llama.c:157-166: ffn_gate_inp + per-expert tensors).
 *
 * gate_inp : router weights, fp32 [NE][E] (tensor gate_inp->data).
 * gate_e, up_e : NE base pointers, each to EI rows of E columns (blocks).
 * down_e   : NE base pointers, each to E rows of EI columns (blocks).
 *            For OLMoE's stacked tensors pass base + e * expert_bytes, exactly
 *            the view tensor_at_q (olmoe.c:20-60) forms; for Mixtral pass
 *            hl->gate_exp[e]->qdata etc.
 * wtype    : HIP_MOE_Q8_0 or HIP_MOE_Q4_0 (all three matrices the same type).
 * topk     : experts per token (1 <= topk <= NE <= 256).
 * renorm   : 0 = OLMoE (weights are the softmax probabilities),
 *            1 = Mixtral (weights divided by their sequential sum, llama.c:422-427).
 * E and EI must be multiples of 256.
 *
 * Host buffers are only read; the caller keeps ownership (GGUF mmap views).
 * Returns NULL if not applicable (no device, unsupported type/shape, OOM).
 */
hip_moe_layer *hip_moe_upload(const float *gate_inp,
                              const void *const *gate_e,
                              const void *const *up_e,
                              const void *const *down_e,
                              int wtype, size_t E, size_t EI, size_t NE,
                              size_t topk, int renorm);

/*
 * The same with the gate/up and down block types given apart, as the
 * reference's tensors carry them (hl->gate_exps->type, hl->down_exps->type):
 * a Q4_K_M GGUF keeps gate/up in Q4_K and down in Q6_K or Q4_K.  Q8_0/Q4_0
 * need gate_type == down_type (then this is hip_moe_upload).  K-quant
 * experts (gate/up and down each HIP_MOE_Q4_K or HIP_MOE_Q6_K; E a multiple
 * of 256 up to 8192, EI up to 16384) stay as the tensors' rows and take one
 * path for every T: routing, then per (token, slot) the Q8_K integer
 * gate/up dots of the reference's -DQ8_DOT build, SwiGLU, and the fp32 down
 * dot in the reference's own order (fused_ffn_silu, nn.c:449-539), then the
 * combine; outputs, ids and weights equal the reference's bit for bit.
 */
hip_moe_layer *hip_moe_upload_typed(const float *gate_inp,
                                    const void *const *gate_e,
                                    const void *const *up_e,
                                    const void *const *down_e,
                                    int gate_type, int down_type, size_t E, size_t EI,
                                    size_t NE, size_t topk, int renorm);

/*
 * out[T][E] = moe_ffn(x[T][E]), synchronous, host fp32 buffers (the contract
 * of moe_ffn(model, input, output, l): output is overwritten, olmoe.c:357).
 *
 * router_bias : optional fp32 [NE] added to every token's router logits
 *               first, as the reference's add argument of
 *               tensor_mma_transposed_2x2 does (matmul.c:13-33): logit =
 *               bias + dot.  NULL = no bias (what moe_ffn passes).
 * ids_out     : optional [T][topk] expert ids, ascending weight (top_k order).
 * w_out       : optional [T][topk] routing weights (after renorm if enabled).
 * Returns 1 on success, 0 if not applicable.
 */
int hip_moe_ffn(hip_moe_layer *L, const float *x, float *out, size_t T,
                const float *router_bias, uint32_t *ids_out, float *w_out);

/*
 * Same as hip_moe_ffn with every pointer in device memory, enqueued on
 * `stream` (a hipStream_t) without waiting.  NULL = the library's stream for
 * the current device, shared by every layer, so calls without a stream run
 * in call order.  This is the form a device-resident forward pass (and a
 * HIP graph) uses.
 *
 * The decode path (T*topk <= 64) is one persistent launch that keeps a
 * workgroup on every CU, and its workgroups wait on one another: do not
 * let two such calls run at once on different streams (order them by
 * stream or event).  Overlapping ones can each hold CUs the other needs;
 * they end on bounded waits and set the layer's error word.  The error is
 * sticky: from then on every decode call of the layer writes NaN outputs
 * (ids 0, weights NaN) until hip_moe_status (or the synchronous
 * hip_moe_ffn) reports it and resets the layer.
 *
 * Scratch grows to the largest T seen.  A call that would grow it while
 * `stream` is being captured into a HIP graph returns 0 (growth frees
 * buffers the graph would name): call hip_moe_reserve before capturing.
 */
int hip_moe_ffn_dev(hip_moe_layer *L, const float *d_x, float *d_out, size_t T,
                    const float *d_router_bias, uint32_t *d_ids_out,
                    float *d_w_out, void *stream);

/*
 * hip_moe_ffn_dev without allocating: the decode path only (T*topk <= 64,
 * where hip_moe_path_for gives HIP_MOE_PATH_DECODE or the path is forced to
 * it), its scratch (sync words, tagged partials, and ids/weights when
 * d_ids_out/d_w_out are NULL) in a static device array of 12 MiB per GPU,
 * set up by the first hip_moe_upload on that GPU.  It calls no hipMalloc,
 * hipFree, memset or synchronisation, so it can be captured into a HIP
 * graph with no reserve step.  A call whose scratch would exceed the array
 * returns 0 with an error.  Every call on one GPU shares the array: calls
 * that overlap on one GPU (two streams, any layers) race.  An expired wait
 * is sticky as on hip_moe_ffn_dev; hip_moe_status on any layer of that GPU
 * reports and clears it.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under graph capture, serving loops, harnesses that forbid it).
 */
int hip_moe_ffn_dev_noalloc(hip_moe_layer *L, const float *d_x, float *d_out, size_t T,
                            const float *d_router_bias, uint32_t *d_ids_out,
                            float *d_w_out, void *stream);

/*
 * Size the layer's scratch for calls of up to T tokens now (synchronous).
 * No counterpart in the reference (its scratch tensors are sized at load,
 * olmoe.c:185-199); device-pointer and graph callers use it so that no call
 * allocates later.  1 = ok.
 */
int hip_moe_reserve(hip_moe_layer *L, size_t T);

/*
 * Wait for `stream` (NULL = the library's stream) and report whether a
 * bounded wait of the decode kernel ran out since the last report (in the
 * layer's scratch, or in the static scratch of its GPU):
 * 0 = no, 1 = router logits, 2 = partial sums, 3 = start flags, -1 = the
 * query failed.  On an error it also resets the layer's sync words, so
 * later calls compute again; the outputs of the failed call and of every
 * call since were invalid.  The reference has no asynchronous entry point
 * and no counterpart; hip_moe_ffn runs this check itself.
 */
int hip_moe_status(hip_moe_layer *L, void *stream);

/*
 * Diagnostic: bound every wait of the layer's decode kernel at `polls`
 * poll rounds (0 = the default, 2^20).  Tests force the error path with a
 * tiny bound; every wait still ends and the kernel exits normally.  No
 * counterpart in the reference.  1 = ok.
 */
int hip_moe_set_wait_limit(hip_moe_layer *L, int polls);

/*
 * Routing stage alone, device pointers, enqueued on `stream`:
 * router logits (matmul.c:270-324), softmax_1d (nn.c:221-262), top_k
 * (nn.c:276-308) and the Mixtral renormalisation (llama.c:422-427).
 * d_logits [T][NE] receives the raw logits and d_probs [T][NE] the softmax
 * probabilities (either may be NULL); d_ids/d_w [T][topk] are required.
 */
int hip_moe_route_dev(hip_moe_layer *L, const float *d_x, size_t T,
                      const float *d_router_bias, float *d_logits,
                      float *d_probs, uint32_t *d_ids, float *d_w,
                      void *stream);

/*
 * One expert for one token, device pointers: out[E] = down_e .
 * (silu(gate_e . x) * (up_e . x)).  The per-expert body of moe_ffn, i.e.
 * fused_ffn_silu (nn.c:496-539) on the views tensor_at_q forms.
 */
int hip_moe_expert_ffn_dev(hip_moe_layer *L, size_t expert, const float *d_x,
                           float *d_out, void *stream);

/*
 * Execution paths of hip_moe_ffn / hip_moe_ffn_dev.  None has a counterpart
 * in the reference, which runs one per-token loop (olmoe.c:364-406):
 *   DECODE   one persistent launch (T*k <= 64, NE <= 64), fp32 arithmetic
 *   GEMV     router, top-k, per-pair dequant-GEMV kernels, combine; fp32
 *   GROUPED  router, top-k, sort by expert, f16 MFMA grouped GEMMs, combine
 * AUTO picks DECODE where it applies and the (token, slot) pairs stay at
 * 3/4 of the experts (4*T*k <= 3*NE: OLMoE T <= 6, Mixtral T <= 3; every
 * pair streams its expert once), else GROUPED (each touched expert streamed
 * once), else GEMV.  Routing (ids and
 * weights) is bit-identical on every path; outputs agree with the reference
 * within 1e-3 relative L2 (fp32 paths: ~1e-6; GROUPED: ~5e-4 from f16
 * operands).
 */
#define HIP_MOE_PATH_AUTO 0
#define HIP_MOE_PATH_DECODE 1
#define HIP_MOE_PATH_GEMV 2
#define HIP_MOE_PATH_GROUPED 3

/* Force a path for later calls (AUTO restores the default); 1 = ok.  A
 * forced path that does not apply to a call makes that call return 0. */
int hip_moe_set_path(hip_moe_layer *L, int path);

/* The path a call with T tokens takes now, 0 if none applies. */
int hip_moe_path_for(const hip_moe_layer *L, size_t T);

/* Release the device copies and scratch of a layer (NULL is a no-op). */
void hip_moe_free(hip_moe_layer *L);

/* Device bytes held by the layer's weights (router + experts; where the
 * grouped path applies, gate/up are held twice: once as GGML rows for the
 * decode and GEMV kernels, once in the grouped GEMMs' row-group layout). */
size_t hip_moe_weight_bytes(const hip_moe_layer *L);

/* The last error message of this library ("" if none). */
const char *hip_moe_last_error(void);

/*
 * expf as the device evaluates it inside softmax and SwiGLU, over n floats
 * in device memory.  It has no counterpart in the reference; it exists so the
 * device function can be compared with the host's glibc expf (which the
 * reference calls, vector_avx2.h:50-63) over every input.
 */
int hip_moe_expf_dev(const float *d_in, float *d_out, size_t n, void *stream);

/*
 * A plain streaming copy of `bytes` (a multiple of 16) between device
 * buffers, with 16-byte loads and stores.  It has no counterpart in the
 * reference: profilers read its HBM byte counters (bytes read and written
 * known exactly) to calibrate the counters of the MoE kernels.
 */
int hip_moe_copy_dev(const void *d_src, void *d_dst, size_t bytes, void *stream);

/*
 * Dense quantized matrices: the reference's tensor_mma_transposed_2x2 with a
 * Q8_0/Q4_0 right operand (matmul.c:451-462 -> 270-324), as its models use
 * it for the attention projections (olmoe.c:448-450, llama.c:498-505), the
 * output projection and the lm_head (olmoe.c:563,577), and its fused_gemv2/3
 * (nn.c:399-425: one such product per weight segment, which map to calls in
 * a row on one stream).
 *
 * hip_moe_qmat_upload copies one matrix of N rows of K columns (the tensor's
 * qdata: GGUF blocks, row-major) to the current device, once, unchanged.
 * Q8_0/Q4_0: K/64 must be a power of two from 4 to 64 (K = 256 .. 4096:
 * OLMoE 2048, Mixtral 4096).  Q4_K/Q6_K: K a multiple of 256 up to 32768
 * (Mixtral's 14336 included).  NULL if not applicable.
 */
typedef struct hip_moe_qmat hip_moe_qmat;

hip_moe_qmat *hip_moe_qmat_upload(const void *qdata, int wtype, size_t N, size_t K);

/*
 * out[T][N] = add + x[T][K] . W^T, host fp32 buffers, synchronous:
 * tensor_mma_transposed_2x2(out, x, W, add).  As mma_init (matmul.c:13-33)
 * does, add holds add_len = T*N values (one per output) or N (the same row
 * for every token), or is NULL (zero); any other add_len returns 0.  Each
 * output is fl(add + dot), the dot in fp32 in another order than the
 * reference's dot_f32_quant (which its default -DQ8_DOT build takes for
 * every T: matmul.c:107-131,145-165,285-312, quant.c:656-668), each block
 * as d * (sum((q + c) x) - c * sum(x)), c = 128 (Q8_0) or 8 (Q4_0):
 * absolute error per output within 2^-24 * (32 (127 + c) + 31 c + 64 * 255)
 * * (sum over blocks of |d| * sum |x|) to first order; ~1e-6 relative L2 on
 * zero-mean activations.  Several tokens (T >= 2) of a Q8_0/Q4_0 matrix run
 * on the matrix cores instead: each 32-value token block scaled by a power
 * of two and split into two f16 parts (~22 bits together), the quants
 * unscaled (exact in f16), the block scale applied per block in fp32, so the
 * outputs keep fp32 accuracy (~1e-7 relative, summation order only).
 * Q4_K/Q6_K matrices take the reference's Q8_K
 * path (matmul.c:291-297: each token quantized by quantize_row_q8, then
 * dot_q4_K_q8_K / dot_q6_K_q8_K, quant_avx2.h:8-209): there every output
 * equals the reference's bit for bit (the integer sums are exact and the
 * fp32 steps are the reference's, in its order).  Returns 1 on success, 0
 * if not applicable.
 */
int hip_moe_qmat_mul(hip_moe_qmat *W, const float *x, size_t T, const float *add,
                     size_t add_len, float *out);

/* The same on device pointers (d_x 16-byte aligned), enqueued on `stream`
 * without waiting (NULL = the library's stream for W's device).  It
 * allocates nothing: the matrix-core form's token buffer, made at upload,
 * holds 64 tokens (more after a host call of more tokens); calls with more
 * take the per-token product.  Calls that overlap on one matrix race on
 * that buffer.  A host call (hip_moe_qmat_mul) with more tokens than the
 * buffer holds replaces it (after waiting for the device): HIP graphs
 * captured earlier with this function on W name the freed buffer and must
 * be captured again. */
int hip_moe_qmat_mul_dev(const hip_moe_qmat *W, const float *d_x, size_t T,
                         const float *d_add, size_t add_len, float *d_out, void *stream);

/* Device bytes of the matrix's blocks. */
size_t hip_moe_qmat_bytes(const hip_moe_qmat *W);

/*
 * quantize_row_q8 (quant.c:627-654) of T rows of K values on the current
 * device, bit for bit: d[T][K/256] scales, qs[T][K] quants, bsums
 * [T][K/256][16] sums of 16 quants (block_q8_K's fields, quant.h:80-85,
 * unpacked).  The step the K-quant products run on their tokens, exposed
 * for checking.  K a multiple of 256; x 16-byte and qs 4-byte aligned.
 */
int hip_moe_quantize_q8k_dev(const float *d_x, size_t T, size_t K, float *d_d, int8_t *d_qs,
                             int16_t *d_bsums, void *stream);

/* Release the device copy (NULL is a no-op). */
void hip_moe_qmat_free(hip_moe_qmat *W);

#ifdef __cplusplus
}
#endif
#endif
