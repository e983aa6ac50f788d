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

#define LM_HLEN 128   /* head length the attention kernels take */
#define LM_CHUNK 64   /* cache positions per attention workgroup */
#define LM_ARG_NT 1024

/* The step's counters, in device memory, read by every step kernel so that
 * one captured graph serves every step. */
typedef struct LmState {
	int step;     /* steps run since the last reset (prompt + generated) */
	int n_prompt; /* steps that take their token from the prompt */
	int pos;      /* the model's position counter (olmoe.c:95) */
	int size;     /* KV cache rows in use (kvcache.h:14) */
	int tok;      /* the last greedy pick */
	int pad[3];
} LmState;

int lm_launch_embed(int wtype, const uint8_t *wte, int E, const LmState *st, const int *prompt,
                    float *hidden, void *stream);
int lm_launch_add_rmsnorm(const float *a, const float *b, float *h, const float *w, float *x,
                          int E, void *stream);
int lm_launch_qk_rope_kv(float *qkv, const float *q_norm, const float *k_norm,
                         const float *freq, const LmState *st, float *kc, float *vc, int H,
                         int KH, int HL, int C, void *stream);
/* attention partials hold H * lm_attn_chunks(C, window) * (LM_HLEN + 2) floats */
int lm_attn_chunks(int C, int window);
int lm_launch_attention(const float *q, const float *kc, const float *vc, const LmState *st,
                        float *part, float *out, int H, int KH, int C, int window,
                        float scale_div, void *stream);
int lm_launch_argmax(const float *logits, int V, LmState *st, int *tokens, void *stream);
int lm_launch_step_end(LmState *st, void *stream);
/* dst[s * slab + i] = src[s * slab + i], i < n, s < slabs (ranges must not
 * overlap within a slab) */
int lm_launch_copy_rows(const float *src, float *dst, size_t slab, size_t n, size_t slabs,
                        void *stream);

#ifdef __cplusplus
}
#endif
#endif
