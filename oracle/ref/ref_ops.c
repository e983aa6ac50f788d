/*
 * TEST INFRASTRUCTURE: thin C entry points over the reference's public
 * functions (tensor_mma_transposed_2x2 matmul.c:451-462, softmax_1d
 * nn.c:221-262, top_k nn.c:276-308, fused_ffn_silu nn.c:496-539,
 * dot_f32_quant quant.c:577-614, quantize_row_q8_0 quant.c:62-78,
 * tensor_mma_transposed_2x2 with a Q8_0/Q4_0 right operand,
 * tensor_div_scalar / tensor_add tensor.c:334-353,435-456, quantize_row_q8
 * and dot_q8_quant quant.c:627-668, dequant_row quant.c:533-575), linked against
 * the reference's own objects.  ref_moe_ffn_composed runs moe_ffn's loop
 * (olmoe.c:355-406, llama.c:407-456) over those functions with the router
 * bias passed through tensor_mma_transposed_2x2's add argument; with a NULL
 * bias it must equal the reference's static moe_ffn bit for bit.
 */
#include "tensor.h"
#include "matmul.h"
#include "nn.h"
#include "quant.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* expert block types: wtype holds the gate/up type, or'ed with the down
 * type << 8 where that differs */
#define WT_GU(w) ((w) & 0xff)
#define WT_DN(w) (((w) >> 8) ? ((w) >> 8) : ((w) & 0xff))

static tensor_t *map2(const void *p, size_t d0, size_t d1, int type)
{
	tensor_t *t = tensor_new_mapped((void *)p, d0 * d1, type);
	tensor_reshape_2d(t, d0, d1);
	return t;
}

void ref_route(const float *x, size_t T, size_t E, size_t NE, const float *wr,
	       const float *bias, size_t topk, int renorm, float *logits,
	       float *probs, uint32_t *ids, float *w)
{
	tensor_t *in = map2(x, T, E, TENSOR_F32);
	tensor_t *gi = map2(wr, NE, E, TENSOR_F32);
	tensor_t *add = NULL;
	if (bias) {
		add = tensor_new_mapped((void *)bias, NE, TENSOR_F32);
		tensor_reshape_1d(add, NE);
	}
	tensor_t *gl = tensor_new_zero(2, (size_t)T, (size_t)NE);
	tensor_mma_transposed_2x2(gl, in, gi, add);
	if (logits)
		memcpy(logits, gl->data, T * NE * sizeof(float));
	size_t *idz = malloc(topk * sizeof(size_t));
	float *wv = malloc(topk * sizeof(float));
	for (size_t t = 0; t < T; t++) {
		tensor_t row;
		tensor_at(gl, t, &row);
		softmax_1d(&row);
		if (probs)
			memcpy(&probs[t * NE], row.data, NE * sizeof(float));
		top_k(&row, idz, wv, topk);
		if (renorm) {
			scalar_t s = 0;
			for (size_t e = 0; e < topk; e++)
				s += wv[e];
			for (size_t e = 0; e < topk; e++)
				wv[e] /= s;
		}
		for (size_t e = 0; e < topk; e++) {
			ids[t * topk + e] = (uint32_t)idz[e];
			w[t * topk + e] = wv[e];
		}
	}
	free(idz);
	free(wv);
	tensor_free(gl);
	tensor_free_mapped(in);
	tensor_free_mapped(gi);
	if (add)
		tensor_free_mapped(add);
}

void ref_moe_ffn_composed(const float *x, float *out, size_t T, const float *wr,
			  const float *bias, const void *const *gate_e,
			  const void *const *up_e, const void *const *down_e,
			  int wtype, size_t E, size_t EI, size_t NE, size_t topk,
			  int renorm)
{
	uint32_t *ids = malloc(T * topk * sizeof(uint32_t));
	float *w = malloc(T * topk * sizeof(float));
	ref_route(x, T, E, NE, wr, bias, topk, renorm, NULL, NULL, ids, w);

	tensor_t *eg = tensor_new_zero(2, (size_t)1, (size_t)EI);
	tensor_t *eu = tensor_new_zero(2, (size_t)1, (size_t)EI);
	tensor_t *eo = tensor_new_zero(2, (size_t)1, (size_t)E);
	tensor_t *in = map2(x, T, E, TENSOR_F32);
	tensor_t *o = map2(out, T, E, TENSOR_F32);
	tensor_set(o, 0);
	for (size_t t = 0; t < T; t++) {
		tensor_t tok_in;
		tensor_at(in, t, &tok_in);
		tensor_reshape_2d(&tok_in, 1, E);
		for (size_t e = 0; e < topk; e++) {
			uint32_t id = ids[t * topk + e];
			tensor_t *gw = map2(gate_e[id], EI, E, WT_GU(wtype));
			tensor_t *uw = map2(up_e[id], EI, E, WT_GU(wtype));
			tensor_t *dw = map2(down_e[id], E, EI, WT_DN(wtype));
			int ok = fused_ffn_silu(&tok_in, eo, eg, gw, eu, uw, dw);
			if (!ok)
				abort();
			tensor_t tok_out;
			tensor_at(o, t, &tok_out);
			tensor_reshape_1d(eo, E);
			tensor_div_scalar(eo, eo, 1.0f / w[t * topk + e]);
			tensor_add(&tok_out, &tok_out, eo);
			tensor_reshape_2d(eo, 1, E);
			tensor_free_mapped(gw);
			tensor_free_mapped(uw);
			tensor_free_mapped(dw);
		}
	}
	tensor_free(eg);
	tensor_free(eu);
	tensor_free(eo);
	tensor_free_mapped(in);
	tensor_free_mapped(o);
	free(ids);
	free(w);
}

void ref_fused_ffn(const float *x, const void *gate, const void *up, const void *down,
		   int wtype, size_t E, size_t EI, float *out)
{
	tensor_t *in = map2(x, 1, E, TENSOR_F32);
	tensor_t *eg = tensor_new_zero(2, (size_t)1, (size_t)EI);
	tensor_t *eu = tensor_new_zero(2, (size_t)1, (size_t)EI);
	tensor_t *eo = tensor_new_zero(2, (size_t)1, (size_t)E);
	tensor_t *gw = map2(gate, EI, E, WT_GU(wtype));
	tensor_t *uw = map2(up, EI, E, WT_GU(wtype));
	tensor_t *dw = map2(down, E, EI, WT_DN(wtype));
	if (!fused_ffn_silu(in, eo, eg, gw, eu, uw, dw))
		abort();
	memcpy(out, eo->data, E * sizeof(float));
	tensor_free(eg);
	tensor_free(eu);
	tensor_free(eo);
	tensor_free_mapped(in);
	tensor_free_mapped(gw);
	tensor_free_mapped(uw);
	tensor_free_mapped(dw);
}

float ref_dot(const float *x, const void *qrow, int wtype, size_t n)
{
	return dot_f32_quant(x, qrow, wtype, 0, n);
}

void ref_quantize_q8_0(const float *x, void *blocks, size_t n)
{
	quantize_row_q8_0(x, blocks, n);
}

void ref_expf(const float *in, float *out, size_t n)
{
	for (size_t i = 0; i < n; i++)
		out[i] = expf(in[i]);
}

/* out[T][N] = tensor_mma_transposed_2x2(x[T][K], W[N][K] blocks, add), add
 * NULL, [N] or [T][N] (mma_init matmul.c:13-33) */
void ref_qmat_mul(const float *x, size_t T, const void *q, int wtype, size_t N, size_t K,
		  const float *add, size_t add_len, float *out)
{
	tensor_t *in = map2(x, T, K, TENSOR_F32);
	tensor_t *w = map2(q, N, K, wtype);
	tensor_t *o = map2(out, T, N, TENSOR_F32);
	tensor_t *a = NULL;
	if (add) {
		if (add_len == N) {
			a = tensor_new_mapped((void *)add, N, TENSOR_F32);
			tensor_reshape_1d(a, N);
		} else {
			a = map2(add, T, N, TENSOR_F32);
		}
	}
	tensor_mma_transposed_2x2(o, in, w, a);
	tensor_free_mapped(in);
	tensor_free_mapped(w);
	tensor_free_mapped(o);
	if (a)
		tensor_free_mapped(a);
}

/* quantize_row_q8 (quant.c:627-654), unpacked to d[n/256], qs[n],
 * bsums[n/256][16] */
void ref_quantize_q8k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums)
{
	size_t nb = n / QK_K;
	block_q8_K *y = malloc(nb * sizeof(block_q8_K));
	quantize_row_q8(x, y, n);
	for (size_t i = 0; i < nb; i++) {
		d[i] = y[i].d;
		memcpy(qs + i * QK_K, y[i].qs, QK_K);
		memcpy(bsums + i * 16, y[i].bsums, 16 * sizeof(int16_t));
	}
	free(y);
}

/* dot_q8_quant (quant.c:656-668) of row 0 of qrow with x quantized by
 * quantize_row_q8, as tensor_mma_transposed_2x2 calls it */
float ref_dot_q8k(const float *x, const void *qrow, int wtype, size_t n)
{
	size_t nb = n / QK_K;
	block_q8_K *y = malloc(nb * sizeof(block_q8_K));
	quantize_row_q8(x, y, n);
	float r = dot_q8_quant(y, x, qrow, wtype, 0, n);
	free(y);
	return r;
}

void ref_dequant(const void *qrow, int wtype, float *dst, size_t n)
{
	dequant_row(qrow, wtype, 0, dst, n);
}
