/*
 * Internal interface between the model host layer (hip_lm.c) and the model
 * kernels (lm_kernels.hip).  Launchers return a hipError_t value (0 =
 * success) and enqueue on the given stream without waiting.
 */
#ifndef LM_INTERNAL_H
#define LM_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LM_HLEN 128        /* head length the attention kernel takes */
#define LM_CHUNK 64        /* cache positions per attention workgroup */
#define LM_MAX_CHUNKS 256  /* chunks of one head (context or window <= 16384) */
#define LM_TAG_SLOTS 64    /* gather tags: epoch * 64 + slot */
#define LM_HEAD_SLOT 63    /* the lm_head's slot; layers use 0 .. 62 */
#define LM_MAX_HEAD_WG 4096

#define LM_ERR_GATHER 1    /* a gather's poll ran out */

/* The step's counters in device memory, read by every step kernel so that
 * one captured graph serves every step.  The host writes the first four
 * (it mirrors them exactly); the rest belong to the device. */
typedef struct LmState {
	int step;     /* steps since the run began (prompt + generated) */
	int n_prompt; /* steps that take their token from the prompt */
	int pos;      /* the model's position counter (olmoe.c:95) */
	int size;     /* KV cache rows in use (kvcache.h:14) */
	int tok;      /* the last greedy pick */
	int epoch;    /* steps since upload, never reset: the gathers' tags */
	int err;      /* LM_ERR_* set by a kernel, 0 if none */
	int pad;
} LmState;

/* workgroups of the one-token product kind (0 qkv, 1 output, 2 lm_head)
 * over N rows of K columns: the row groups or what the device holds at
 * once, whichever is fewer; 0 if the shape is not supported */
int lm_gemv_grid(int kind, int wtype, int K, int N);
/* out[N] = rms_norm(a + b) * w . W^T (b may be NULL; a NULL: the step's
 * token row of wte); h_out (may be NULL) receives a + b */
int lm_launch_qkv(int wtype, const uint8_t *W, int N, int K, const float *a, const float *b,
                  const float *w, float *h_out, const uint8_t *wte, const LmState *st,
                  const int *prompt, float *out, int grid, void *stream);
/* attention partials hold H * lm_attn_chunks(C, window) * (LM_HLEN + 2)
 * tagged words; cnt holds H zeroed counters.  nact: the chunks of
 * LM_CHUNK rows covering the step's cache rows (lm_attn_active).  nseq
 * sequences in lockstep: qkv, out, part and cnt hold nseq consecutive
 * copies, and sequence s's cache is kc/vc + s * cstride floats. */
int lm_attn_chunks(int C, int window);
/* which chunk merges a launch's partials: 2 = chunk 0 (the grid KH x nact x
 * nseq is resident at once on the current device), 1 = the last to count in */
int lm_attn_merge_form(int KH, int nact, int nseq);
int lm_launch_attn(const float *qkv, const float *q_norm, const float *k_norm,
                   const float *freq, LmState *st, float *kc, float *vc, uint64_t *part,
                   uint32_t *cnt, float *out, int H, int KH, int C, int window,
                   float scale, int scale_mul, int layer, int nact, int nseq,
                   size_t cstride, void *stream);

/* out[K] = the dequantized token_embd row of the step's token (wtype 1
 * Q8_0, 2 Q4_0, 3 Q4_K, 5 Q6_K) */
int lm_launch_embed(int wtype, const uint8_t *wte, int K, const LmState *st, const int *prompt,
                    float *out, void *stream);

/* prefill of T prompt rows of nseq sequences (rows z * T + t) at cache row
 * `size` and position pos0 (size + T <= C): q/k norms (q_norm and k_norm
 * both NULL for Mixtral) and RoPE of the stacked q/k/v rows, q into qo
 * [nseq * T][H * 128], k and v into the cache rows size .. size + T - 1 */
int lm_launch_pf_qk(const float *qkv, const float *q_norm, const float *k_norm,
                    const float *freq, float *kc, float *vc, float *qo, int H, int KH, int C,
                    int size, int pos0, int T, int nseq, size_t cstride, void *stream);
/* causal (and sliding-window) attention of those rows over the cache rows
 * 0 .. size + T - 1 into out [nseq * T][H * 128] */
int lm_launch_pf_attn(const float *qo, const float *kc, const float *vc, float *out, int H,
                      int KH, int C, int size, int T, int window, float scale, int scale_mul,
                      int nseq, size_t cstride, void *stream);

/* h_out[s] = add[s] + the KS partial-sum slices (TN floats apart) of a
 * matrix-core product added in stretch order (k_qmm_reduce's sum) and x_out[s]
 * = rms_norm(h_out[s]) * w, for the nseq rows of E floats: the product's
 * reduce and the row norm as one launch, with the same bits */
int lm_launch_norm_parts(int nseq, int E, const float *part, int KS, size_t TN,
                         const float *add, const float *w, float *h_out, float *x_out,
                         void *stream);

/* chunks a step over a cache of `size` rows (before the step) reads */
static inline int lm_attn_active(int size, int window)
{
	const int AT = size + 1, lo = window > 0 && AT > window ? AT - window : 0;
	return (AT - lo + LM_CHUNK - 1) / LM_CHUNK;
}
/* out[N] = add + x . W^T, then x_out = rms_norm(out) * w (rows_t: N tagged
 * words, cnt one zeroed counter) */
int lm_launch_oproj(int wtype, const uint8_t *W, int N, int K, const float *x,
                    const float *add, float *out, uint64_t *rows_t, const float *w,
                    float *x_out, LmState *st, int layer, int grid, void *stream);
/* logits out[N] = rms_norm(a + b) * w . W^T, the greedy pick and the
 * counters' advance (best: 2 * grid tagged words, cnt one zeroed counter) */
int lm_launch_head(int wtype, const uint8_t *W, int N, int K, const float *a, const float *b,
                   const float *w, float *out, uint64_t *best, LmState *st, int *tokens,
                   int grid, void *stream);
int lm_launch_step_end(LmState *st, void *stream);
/* nseq sequences in lockstep: x_out[s] = rms_norm(a[s] + b[s]) * w (b may
 * be NULL; a NULL: the embedding row of sequence s's step token, from
 * prompt[s][step] while the prompt lasts, then btok[s]); h_out[s] (may be
 * NULL) receives a[s] + b[s] */
int lm_launch_norm_rows(int wtype, int nseq, int E, const float *a, const float *b,
                        const float *w, float *h_out, float *x_out, const uint8_t *wte,
                        const LmState *st, const int *prompt, const int *btok, void *stream);
/* btok[s] = the first maximum of logits[s][V], also into
 * tokens[s * tstride + step] (tokens may be NULL) */
int lm_launch_pick_rows(const float *logits, int nseq, int V, const LmState *st, int *btok,
                        int *tokens, int tstride, void *stream);
/* dst[s * slab + i] = src[s * slab + i], i < n, s < slabs (ranges must not
 * overlap within a slab) */
int lm_launch_copy_rows(const float *src, float *dst, size_t slab, size_t n, size_t slabs,
                        void *stream);

#ifdef __cplusplus
}
#endif
#endif
