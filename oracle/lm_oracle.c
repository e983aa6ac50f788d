/*
 * CPU oracle for the OLMoE model around the MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP model kernels, loaded by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py; the
 * product library never links or calls it.
 *
 * A plain-C restatement of the reference's OLMoE decode step
 * (models/olmoe/olmoe.c:409-520, AVX2 build) over the MoE oracle of
 * moe_oracle.c.  Compiled -ffp-contract=off: each fused multiply-add the
 * reference's clang build forms (vector_fma, and the a*b+c expressions its
 * default -ffp-contract=on contracts, left operand first) is written as
 * fmaf; every other product and sum rounds on its own.
 *
 * Parity pins (tests/test_oracle.py): per-step logits and greedy tokens
 * bit-for-bit against the compiled reference's own olmoe_decode /
 * olmoe_prefill driven by oracle/ref/ref_olmoe.c (tests/golden/
 * olmoe_model_*.npz), on a reduced model with non-unit norms and at the
 * full shape; RMSNorm and RoPE also against float64 closed forms.
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define LANES 8

struct orc_olmoe {
	size_t L, E, H, HLEN, V, NE, K, EI, C;
	float theta, hlen_sq;
	int wtype;
	const void *const *p; /* the caller's pointer table */
	size_t size;          /* kvcache size (kvcache.h:14) */
	int pos;              /* the model's position counter (olmoe.c:95) */
	float *kc, *vc;       /* [L][H][C][HLEN] */
	float *hidden, *x, *q, *k, *v, *attn, *out, *resid, *moe_in, *scores;
	const void **ge, **ue, **de; /* [NE] expert views of one layer */
};

static size_t qrow_bytes(int wtype, size_t n)
{
	return n / 32 * (wtype == ORC_Q8_0 ? 34 : 18);
}

/* vector_avx2.h:126-132 */
static float tree8(const float a[LANES])
{
	float v0 = a[0] + a[4], v1 = a[1] + a[5], v2 = a[2] + a[6], v3 = a[3] + a[7];
	return (v0 + v2) + (v1 + v3);
}

/*
 * rms_norm (nn.c:8-51) of one row: lane sums of x*x (product, then sum),
 * the tree, an FMA scalar tail, rms = sqrtf(sum / len + 1e-5f), x / rms,
 * then tensor_mul by the weight (tensor.c:393-412).
 */
static void rms_norm_row(float *dst, const float *src, const float *w, size_t n)
{
	float s[LANES] = {0};
	size_t nv = n - n % LANES;
	for (size_t i = 0; i < nv; i += LANES)
		for (int l = 0; l < LANES; l++) {
			float sq = src[i + l] * src[i + l];
			s[l] = s[l] + sq;
		}
	float sum = tree8(s);
	for (size_t i = nv; i < n; i++)
		sum = fmaf(src[i], src[i], sum);
	float rms = sqrtf(sum / (float)n + 1e-5f);
	for (size_t i = 0; i < n; i++) {
		float r = src[i] / rms;
		dst[i] = r * w[i];
	}
}

/* rope_apply (nn.c:192-219) on H heads of HLEN: consecutive pairs (2i, 2i+1) */
static void rope(float *t, size_t H, size_t HLEN, int pos, float theta)
{
	size_t half = HLEN / 2;
	for (size_t h = 0; h < H; h++) {
		float *head = t + h * HLEN;
		for (size_t i = 0; i < half; i++) {
			float freq = 1.0f / powf(theta, (float)(2 * i) / (float)HLEN);
			float angle = (float)pos * freq;
			float c = cosf(angle), s = sinf(angle);
			float x0 = head[2 * i], x1 = head[2 * i + 1];
			head[2 * i] = fmaf(x0, c, -(x1 * s));
			head[2 * i + 1] = fmaf(x0, s, x1 * c);
		}
	}
}

/* kvcache_rotate (kvcache.c:31-56): keep the last C/2 entries */
static void kv_rotate(orc_olmoe *m)
{
	size_t keep = m->C / 2;
	if (keep > m->size)
		keep = m->size;
	size_t drop = m->size - keep;
	for (size_t i = 0; i < m->L * m->H; i++) {
		float *kb = m->kc + i * m->C * m->HLEN, *vb = m->vc + i * m->C * m->HLEN;
		memmove(kb, kb + drop * m->HLEN, keep * m->HLEN * sizeof(float));
		memmove(vb, vb + drop * m->HLEN, keep * m->HLEN * sizeof(float));
	}
	m->size = keep;
}

orc_olmoe *orc_olmoe_new(size_t layers, size_t E, size_t H, size_t V, size_t NE, size_t topk,
			 size_t EI, size_t C, float theta, int wtype, const void *const *ptrs)
{
	orc_olmoe *m = calloc(1, sizeof(*m));
	if (!m)
		return NULL;
	m->L = layers;
	m->E = E;
	m->H = H;
	m->HLEN = E / H;
	m->V = V;
	m->NE = NE;
	m->K = topk;
	m->EI = EI;
	m->C = C;
	m->theta = theta;
	m->hlen_sq = (float)sqrt((double)(float)m->HLEN); /* olmoe.c:150 */
	m->wtype = wtype;
	m->p = ptrs;
	m->kc = calloc(layers * H * C * m->HLEN, sizeof(float));
	m->vc = calloc(layers * H * C * m->HLEN, sizeof(float));
	float **bufs[] = {&m->hidden, &m->x, &m->q, &m->k, &m->v, &m->attn, &m->out,
			  &m->resid, &m->moe_in};
	for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
		*bufs[i] = calloc(E, sizeof(float));
	m->scores = calloc(C, sizeof(float));
	m->ge = calloc(NE, sizeof(void *));
	m->ue = calloc(NE, sizeof(void *));
	m->de = calloc(NE, sizeof(void *));
	return m;
}

void orc_olmoe_free(orc_olmoe *m)
{
	if (!m)
		return;
	free(m->kc);
	free(m->vc);
	free(m->hidden);
	free(m->x);
	free(m->q);
	free(m->k);
	free(m->v);
	free(m->attn);
	free(m->out);
	free(m->resid);
	free(m->moe_in);
	free(m->scores);
	free(m->ge);
	free(m->ue);
	free(m->de);
	free(m);
}

/*
 * transformer() in decode mode (olmoe.c:214-341) for layer l: each head's
 * k and v go to cache row `size`; scores = q . K^T (the GEMV of matmul.c:
 * 115-118, one dot_f32_f32 each), / hlen_sq (tensor_div_scalar), softmax_1d,
 * then P . V (nontrans_thread_fn, matmul.c:56-69: per output column an FMA
 * chain over the positions in order, seeded with 0).
 */
static void attention(orc_olmoe *m, size_t l)
{
	const size_t H = m->H, HL = m->HLEN, C = m->C, AT = m->size + 1;
	for (size_t h = 0; h < H; h++) {
		float *K = m->kc + (l * H + h) * C * HL, *Vv = m->vc + (l * H + h) * C * HL;
		memcpy(K + m->size * HL, m->k + h * HL, HL * sizeof(float));
		memcpy(Vv + m->size * HL, m->v + h * HL, HL * sizeof(float));
		const float *qh = m->q + h * HL;
		for (size_t j = 0; j < AT; j++)
			m->scores[j] = 0.0f + orc_dot_f32(qh, K + j * HL, HL);
		for (size_t j = 0; j < AT; j++)
			m->scores[j] = m->scores[j] / m->hlen_sq;
		orc_softmax_1d(m->scores, AT);
		float *o = m->attn + h * HL;
		for (size_t d = 0; d < HL; d++) {
			float acc = 0.0f;
			for (size_t j = 0; j < AT; j++)
				acc = fmaf(m->scores[j], Vv[j * HL + d], acc);
			o[d] = acc;
		}
	}
}

int orc_olmoe_decode(orc_olmoe *m, int tok, int pos, float *logits, float *trace_moe_in,
		     uint32_t *trace_ids, float *trace_w, int nthreads)
{
	const size_t E = m->E, NE = m->NE, EI = m->EI, K = m->K;
	const int wt = m->wtype;
	/* olmoe_decode (olmoe.c:509-520) */
	if (m->size >= m->C)
		kv_rotate(m);
	if (pos >= (int)m->C)
		pos = (int)m->size;

	orc_dequant_row((const uint8_t *)m->p[0] + (size_t)tok * qrow_bytes(wt, E), wt, m->hidden, E);
	const size_t gu = EI * qrow_bytes(wt, E), dn = E * qrow_bytes(wt, EI);
	for (size_t l = 0; l < m->L; l++) {
		const void *const *p = m->p + 3 + 12 * l;
		rms_norm_row(m->x, m->hidden, (const float *)p[0], E);
		orc_qmat_mul(m->x, 1, p[1], wt, E, E, NULL, 0, m->q);
		orc_qmat_mul(m->x, 1, p[2], wt, E, E, NULL, 0, m->k);
		orc_qmat_mul(m->x, 1, p[3], wt, E, E, NULL, 0, m->v);
		rms_norm_row(m->q, m->q, (const float *)p[4], E);
		rms_norm_row(m->k, m->k, (const float *)p[5], E);
		rope(m->q, m->H, m->HLEN, pos, m->theta);
		rope(m->k, m->H, m->HLEN, pos, m->theta);
		attention(m, l);
		orc_qmat_mul(m->attn, 1, p[6], wt, E, E, NULL, 0, m->out);
		for (size_t i = 0; i < E; i++) { /* tensor_add (tensor.c:334-353) */
			m->hidden[i] = m->hidden[i] + m->out[i];
			m->resid[i] = m->hidden[i];
		}
		rms_norm_row(m->moe_in, m->hidden, (const float *)p[7], E);
		if (trace_moe_in)
			memcpy(trace_moe_in + l * E, m->moe_in, E * sizeof(float));
		for (size_t e = 0; e < NE; e++) { /* tensor_at_q (olmoe.c:20-60) */
			m->ge[e] = (const uint8_t *)p[9] + e * gu;
			m->ue[e] = (const uint8_t *)p[10] + e * gu;
			m->de[e] = (const uint8_t *)p[11] + e * dn;
		}
		orc_moe_ffn(m->moe_in, m->out, 1, (const float *)p[8], NULL, m->ge, m->ue, m->de, wt,
			    E, EI, NE, K, 0, trace_ids ? trace_ids + l * K : NULL,
			    trace_w ? trace_w + l * K : NULL, NULL, NULL, nthreads);
		for (size_t i = 0; i < E; i++)
			m->hidden[i] = m->resid[i] + m->out[i];
	}
	m->size++;
	rms_norm_row(m->x, m->hidden, (const float *)m->p[2], E);
	float *lg = logits ? logits : malloc(m->V * sizeof(float));
	orc_qmat_mul(m->x, 1, m->p[1], wt, m->V, E, NULL, 0, lg);
	size_t best = 0;
	for (size_t i = 1; i < m->V; i++)
		if (lg[i] > lg[best])
			best = i;
	if (!logits)
		free(lg);
	return (int)best;
}

void orc_olmoe_run(orc_olmoe *m, const int *prompt, size_t n_prompt, size_t n_gen,
		   float *logits, int *tokens, int nthreads)
{
	int tok = 0;
	for (size_t i = 0; i < n_prompt; i++)
		tok = orc_olmoe_decode(m, prompt[i], m->pos++, i + 1 == n_prompt ? logits : NULL,
				       NULL, NULL, NULL, nthreads);
	tokens[0] = tok;
	for (size_t s = 1; s <= n_gen; s++) {
		tok = orc_olmoe_decode(m, tok, m->pos++, logits ? logits + s * m->V : NULL, NULL,
				       NULL, NULL, nthreads);
		tokens[s] = tok;
	}
}
