/*
 * hip_lm.h - C ABI of the MI355X (gfx950) whole-model decode around the
 * quantized MoE layer: an OLMoE- or Mixtral-shaped transformer run one token
 * at a time on one GPU, weights resident in HBM in their GGUF blocks,
 * activations and the fp32 KV cache resident too.
 *
 * Drop-in for the decode side of the reference's model plugins:
 *   olmoe_load / olmoe_decode / olmoe_generate / olmoe_close
 *     (models/olmoe/olmoe.c:123-201, 409-520, 522-600, 602-645)
 *   and the greedy pick of main.c:189-193.
 * One step is the reference's olmoe_forward for one token (olmoe.c:409-500):
 * embedding, per layer RMSNorm, q/k/v products, q/k RMSNorm (OLMoE), RoPE,
 * attention over the KV cache (olmoe.c:214-341, kvcache.c), output product
 * and residual, RMSNorm, moe_ffn (hip_moe.h), residual; then the final
 * RMSNorm, the lm_head product (olmoe.c:558-564) and the greedy pick.
 *
 * Conventions as hip_moe.h: plain C, pointers and sizes; 1 = done, 0 = not
 * applicable or failed (message in hip_moe_last_error()); nothing exits.
 * Arithmetic is fp32 throughout (dots in another order than the
 * reference's): per-step logits agree with the reference's within 1e-3
 * relative L2.
 */
#ifndef HIP_LM_H
#define HIP_LM_H

#include <stddef.h>
#include <stdint.h>

#include "hip_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HIP_LM_OLMOE 1   /* q/k full-vector RMSNorm, softmax top-k without renorm */
#define HIP_LM_MIXTRAL 2 /* grouped-query attention, renormalised top-k */

/*
 * The model's tensors as the reference's loader maps them (gguf.c views of
 * the GGUF file; the caller keeps ownership, they are only read):
 * quantized matrices are rows of GGUF blocks of type wtype (HIP_MOE_Q8_0,
 * HIP_MOE_Q4_0, HIP_MOE_Q4_K or HIP_MOE_Q6_K) unless the per-tensor types
 * below say otherwise, norms and the router fp32.  A model whose matrices
 * are all Q8_0 or all Q4_0 runs the fused step kernels; any other mix runs
 * a step of separate norm, product and attention launches (the K-quant
 * products through Q8_K activations, bit for bit the reference's dots).  Per-layer arrays hold `layers`
 * pointers; the expert arrays hold layers * NE pointers (layer-major), each
 * the base of one expert's matrix: for OLMoE's stacked *_exps tensors base +
 * e * expert_bytes (tensor_at_q, olmoe.c:20-60), for Mixtral the per-expert
 * tensors (llama.c:157-166).
 */
typedef struct hip_lm_desc {
	int arch;                 /* HIP_LM_OLMOE or HIP_LM_MIXTRAL */
	int wtype;                /* block type of every quantized matrix */
	size_t layers, E, heads, kv_heads, vocab, context, NE, topk, EI;
	float rope_theta;
	size_t sliding_window;    /* 0 = full attention */
	const void *token_embd;   /* [vocab][E] */
	const void *output;       /* lm_head [vocab][E] */
	const float *output_norm; /* [E] */
	const float *const *attn_norm;                /* [E] */
	const void *const *attn_q;                    /* [heads * 128][E] */
	const void *const *attn_k, *const *attn_v;    /* [kv_heads * 128][E] */
	const void *const *attn_o;                    /* [E][heads * 128] */
	const float *const *q_norm, *const *k_norm;   /* OLMoE [E]; NULL otherwise */
	const float *const *ffn_norm;                 /* [E] */
	const float *const *gate_inp;                 /* router [NE][E] */
	const void *const *gate_e, *const *up_e;      /* [layers * NE]: [EI][E] each */
	const void *const *down_e;                    /* [layers * NE]: [E][EI] each */
	/* Block types per tensor, as the reference's tensors carry them
	 * (tensor->type; a Q4_K_M GGUF mixes Q4_K and Q6_K): 0 = wtype.
	 * layer_types (NULL = wtype everywhere) holds [layers][6]: attn_q,
	 * attn_k, attn_v, attn_output, the experts' gate/up, the experts' down.
	 * Each of HIP_MOE_Q8_0, Q4_0, Q4_K, Q6_K (K-quant tensors: E, heads *
	 * 128 and EI multiples of 256); wtype itself may be Q4_K or Q6_K. */
	int embd_type, output_type;
	const int *layer_types;
} hip_lm_desc;

typedef struct hip_lm hip_lm;

/*
 * Upload every tensor to the current device once and allocate the KV cache
 * (layers x kv_heads x context x 128 fp32 for k and for v) and the step's
 * buffers.  Replaces olmoe_load's residency (olmoe.c:123-201).  Head length
 * must be 128; E, heads*128 and EI must suit hip_moe_upload and
 * hip_moe_qmat_upload.  NULL if not applicable.
 */
hip_lm *hip_lm_upload(const hip_lm_desc *d);

/*
 * One step at the model's position (olmoe_decode(model, tok, model->pos)
 * then model->pos++, olmoe.c:509-520, with kvcache_rotate when the cache is
 * full), then the lm_head product: logits[vocab] (host, optional) and the
 * greedy pick *next (optional).  Synchronous.
 */
int hip_lm_decode(hip_lm *M, int tok, float *logits, int *next);

/*
 * olmoe_prefill / llama_prefill (olmoe.c:504-508, llama.c:560-564): the n
 * prompt ids as one forward at the model's position (causal attention over
 * the cache and the new rows; every layer on n rows), then the lm_head
 * product of the last row: logits[vocab] (host, optional) and the greedy
 * pick *next (optional), which the next hip_lm_decode does not need (pass
 * it as that step's token).  The cache grows by n rows; the ids must fit
 * (cache rows in use + n <= context; the reference's prefill does not
 * rotate and writes past its cache otherwise): 0 with an error if not.
 * Synchronous.
 */
int hip_lm_prefill(hip_lm *M, const int *prompt, size_t n, float *logits, int *next);

/*
 * olmoe_generate without tokenizer and EOS stop (olmoe.c:522-600): the
 * prompt as one prefill (as hip_lm_prefill; a prompt of one id, or one that
 * does not fit the cache, runs one step per id instead), then n_gen greedy
 * steps; tokens[0..n_gen] are the n_gen + 1 picks (after the prompt, and
 * after each generated token).  Every step runs from device memory (token,
 * position and cache row are device counters; steps replay captured HIP
 * graphs), with no host round trip until the end.  decode_ms (optional):
 * device time of the n_gen generated steps.  Continues from the model's
 * position.
 */
int hip_lm_generate(hip_lm *M, const int *prompt, size_t n_prompt, size_t n_gen, int *tokens,
                    float *decode_ms);

/*
 * The last step's MoE routing, per layer: the router's input moe_in
 * [layers][E] (the pre-MoE RMSNorm output), ids and weights [layers][topk].
 * Any pointer may be NULL.  Synchronous.  No counterpart in the reference
 * (its tensor_trace hooks, tensor_trace.c, serve the same purpose).
 */
int hip_lm_trace(hip_lm *M, float *moe_in, uint32_t *ids, float *w);

/*
 * Force every layer's MoE path (HIP_MOE_PATH_*, as hip_moe_set_path; AUTO
 * restores the choice by token count).  A forced path applies to every
 * call, the decode steps' too; HIP_MOE_PATH_GEMV keeps a prefill's MoE
 * layers in fp32 where the grouped path's f16 operands would move them by
 * ~5e-4.  The model's lockstep batches take it as well.  No counterpart
 * in the reference.  1 = ok.
 */
int hip_lm_set_moe_path(hip_lm *M, int path);

/* Empty the KV cache and reset the position (a fresh olmoe_load's state). */
int hip_lm_reset(hip_lm *M);

/* Device bytes of the uploaded weights. */
size_t hip_lm_weight_bytes(const hip_lm *M);

/* Release everything (NULL is a no-op). */
void hip_lm_free(hip_lm *M);

/*
 * Several sequences decoding in lockstep on one model's weights: every step
 * takes one token of each of nseq sequences (the same position in each,
 * their own KV caches), so the weights stream once per step for all of
 * them and the MoE layer runs at T = nseq.  No counterpart in the
 * reference, which decodes one sequence per model (llama.c:578-667, one
 * kvcache); a sequence's results are those of its own single-sequence
 * decode, within the 1e-3 the steps are held to (the MoE layer at T = nseq
 * may take the grouped path, f16 operands).
 *
 * hip_lm_batch_new allocates nseq KV caches (each as hip_lm_upload's) and
 * the step's buffers, and reserves the MoE layers' scratch for T = nseq.
 * It shares M's weights and MoE layers: do not run M and its batches at the
 * same time.  NULL if not applicable.
 */
typedef struct hip_lm_batch hip_lm_batch;

hip_lm_batch *hip_lm_batch_new(hip_lm *M, size_t nseq);

/* One step: toks[nseq] in, logits[nseq][vocab] (host, optional) and the
 * greedy picks next[nseq] (optional) out.  Synchronous. */
int hip_lm_batch_decode(hip_lm_batch *B, const int *toks, float *logits, int *next);

/*
 * hip_lm_generate for every sequence: prompts[nseq][n_prompt] as prefills
 * (each sequence's prompt one forward into its own cache, as
 * hip_lm_prefill; sequences in groups of about 2048 prompt rows per
 * launch; a prompt of one id, or one that does not fit the caches, runs one
 * step per id instead), then n_gen greedy steps; tokens[nseq][n_gen + 1]
 * receive each sequence's picks after its prompt and after each generated
 * token.  Steps replay captured HIP graphs with no host round trip.
 * decode_ms (optional): device time of the n_gen generated steps.  The
 * prefill uses the model's prefill rows: the model and its batches never
 * run at the same time.
 */
int hip_lm_batch_generate(hip_lm_batch *B, const int *prompts, size_t n_prompt, size_t n_gen,
                          int *tokens, float *decode_ms);

/* Empty the caches and reset the position. */
int hip_lm_batch_reset(hip_lm_batch *B);

/* Release the batch (not the model; NULL is a no-op). */
void hip_lm_batch_free(hip_lm_batch *B);

#ifdef __cplusplus
}
#endif
#endif
