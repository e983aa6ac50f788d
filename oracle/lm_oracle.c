/*
 * CPU oracle for the OLMoE and Mixtral models around the MoE FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP model kernels, loaded by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py; the
 * product library never links or calls it.
 *
 * A plain-C restatement of the reference's decode step of OLMoE
 * (models/olmoe/olmoe.c:409-520) and of Mixtral (models/llama/llama.c:
 * 458-576, with its default FLASH_ATTENTION build's flash_attention,
 * nn.c:544-655), AVX2 build, over the MoE oracle of moe_oracle.c.  Compiled -ffp-contract=off: each fused multiply-add the
 * reference's clang build forms (vector_fma, and the a*b+c expressions its
 * default -ffp-contract=on contracts, left operand first) is written as
 * fmaf; every other product and sum rounds on its own.
 *
 * Parity pins (tests/test_oracle_model.py): per-step logits and greedy
 * tokens bit-for-bit against the compiled reference's own olmoe_decode /
 * llama_decode driven by oracle/ref/ref_olmoe.c and ref_llama.c
 * (tests/golden/model_*.npz): reduced models with non-unit norms that run
 * past their context (kvcache_rotate; for Mixtral with a sliding window),
 * the full OLMoE shape, and a two-layer model of the full Mixtral layer
 * shape; with per-tensor block types as a Q4_K_M file mixes them
 * (orc_*_new_typed: Q4_K, Q6_K for the output and some layers' attn_v and
 * experts' down), reduced OLMoE and Mixtral models over 48 positions.
 */
#define _GNU_SOURCE
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define LANES 8

enum { ARCH_OLMOE = 1, ARCH_LLAMA = 2 };

struct orc_lm {
	int arch;
	size_t L, E, QH, KVH, HLEN, V, NE, K, EI, C, window;
	float theta, hlen_sq;
	int *types; /* token_embd, output, then per layer attn_q, attn_k, attn_v,
		     * attn_output, ffn_gate/up_exps, ffn_down_exps */
	const void *const *p; /* the caller's pointer table */
	size_t size;          /* kvcache size (kvcache.h:14) */
	int pos;              /* the model's position counter */
	float *kc, *vc;       /* [L][KVH][C][HLEN] */
	float *hidden, *x, *q, *k, *v, *attn, *out, *resid, *moe_in, *scores;
	const void **ge, **ue, **de; /* [NE] expert views of one layer */
};

struct orc_olmoe {
	struct orc_lm m;
};
struct orc_llama {
	struct orc_lm m;
};

/* bytes of one row of n values in block type t (quant.h:20-78) */
static size_t qrow_bytes(int t, size_t n)
{
	if (t == ORC_Q4_K || t == ORC_Q6_K)
		return n / 256 * (t == ORC_Q4_K ? 144 : 210);
	return n / 32 * (t == ORC_Q8_0 ? 34 : 18);
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

/* kvcache_rotate (kvcache.c:31-56): keep the window, or the last C/2 rows */
static void kv_rotate(struct orc_lm *m)
{
	size_t keep = m->window ? m->window : m->C / 2;
	if (keep > m->size)
		keep = m->size;
	size_t drop = m->size - keep;
	for (size_t i = 0; i < m->L * m->KVH; i++) {
		float *kb = m->kc + i * m->C * m->HLEN, *vb = m->vc + i * m->C * m->HLEN;
		memmove(kb, kb + drop * m->HLEN, keep * m->HLEN * sizeof(float));
		memmove(vb, vb + drop * m->HLEN, keep * m->HLEN * sizeof(float));
	}
	m->size = keep;
}

/* types: 2 + 6 * layers block types (struct orc_lm), or NULL for wtype in
 * every quantized tensor */
static struct orc_lm *lm_new(int arch, size_t layers, size_t E, size_t QH, size_t KVH, size_t V,
			     size_t NE, size_t topk, size_t EI, size_t C, float theta,
			     size_t window, int wtype, const int *types, const void *const *ptrs)
{
	struct orc_lm *m = calloc(1, sizeof(struct orc_olmoe) > sizeof(struct orc_llama)
					     ? sizeof(struct orc_olmoe)
					     : sizeof(struct orc_llama));
	if (!m)
		return NULL;
	m->arch = arch;
	m->L = layers;
	m->E = E;
	m->QH = QH;
	m->KVH = KVH;
	m->HLEN = E / QH;
	m->V = V;
	m->NE = NE;
	m->K = topk;
	m->EI = EI;
	m->C = C;
	m->window = window;
	m->theta = theta;
	m->hlen_sq = (float)sqrt((double)(float)m->HLEN); /* olmoe.c:150, llama.c:118 */
	m->types = malloc((2 + 6 * layers) * sizeof(int));
	if (!m->types) {
		free(m);
		return NULL;
	}
	for (size_t i = 0; i < 2 + 6 * layers; i++)
		m->types[i] = types ? types[i] : wtype;
	m->p = ptrs;
	m->kc = calloc(layers * KVH * C * m->HLEN, sizeof(float));
	m->vc = calloc(layers * KVH * C * m->HLEN, sizeof(float));
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

static void lm_free(struct orc_lm *m)
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
	free(m->types);
	free(m);
}

/* the cache rows of layer l, kv head kh */
static float *kv_rows(const struct orc_lm *m, float *base, size_t l, size_t kh)
{
	return base + (l * m->KVH + kh) * m->C * m->HLEN;
}

/*
 * OLMoE's transformer() in decode mode (olmoe.c:214-341): scores = q . K^T
 * (the GEMV of matmul.c:115-118, one dot_f32_f32 each, seeded with 0),
 * / hlen_sq (tensor_div_scalar), softmax_1d, then P . V
 * (nontrans_thread_fn, matmul.c:56-69: per output column an FMA chain over
 * the positions in order, seeded with 0).
 */
static void attention_olmoe(struct orc_lm *m, size_t l)
{
	const size_t HL = m->HLEN, AT = m->size + 1;
	for (size_t h = 0; h < m->QH; h++) {
		const float *K = kv_rows(m, m->kc, l, h), *Vv = kv_rows(m, m->vc, l, h);
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

/*
 * Mixtral's attention in decode mode (llama.c:238-363 with FLASH_ATTENTION):
 * query head q of kv head q / (QH / KVH), flash_attention (nn.c:544-655) for
 * one row: blocks of 64 positions, s = dot * (1 / hlen_sq), the sliding
 * window's mask (size - kpos >= window), then per block m_new = max(m, block
 * max), correction = expf(m - m_new), o *= correction, l *= correction, and
 * per position p = expf(s - m_new), l += p, o = fma(p, v, o); finally
 * o *= 1 / l.
 */
#define FA_BLOCK 64
static void attention_llama(struct orc_lm *m, size_t l)
{
	const size_t HL = m->HLEN, AT = m->size + 1, G = m->QH / m->KVH;
	const float scale = 1.0f / m->hlen_sq;
	float s[FA_BLOCK];
	for (size_t h = 0; h < m->QH; h++) {
		const size_t kh = h / G;
		const float *K = kv_rows(m, m->kc, l, kh), *Vv = kv_rows(m, m->vc, l, kh);
		const float *qh = m->q + h * HL;
		float *o = m->attn + h * HL;
		float mx = -INFINITY, lsum = 0.0f;
		memset(o, 0, HL * sizeof(float));
		for (size_t j0 = 0; j0 < AT; j0 += FA_BLOCK) {
			const size_t Bk = j0 + FA_BLOCK <= AT ? FA_BLOCK : AT - j0;
			for (size_t j = 0; j < Bk; j++)
				s[j] = orc_dot_f32(qh, K + (j0 + j) * HL, HL) * scale;
			for (size_t j = 0; j < Bk; j++) {
				const size_t kpos = j0 + j;
				if (kpos > m->size)
					s[j] = -INFINITY;
				if (m->window && (int)m->size - (int)kpos >= (int)m->window)
					s[j] = -INFINITY;
			}
			float mi = -INFINITY;
			for (size_t j = 0; j < Bk; j++)
				if (s[j] > mi)
					mi = s[j];
			const float m_new = mx > mi ? mx : mi;
			const float corr = expf(mx - m_new);
			for (size_t d = 0; d < HL; d++)
				o[d] = o[d] * corr;
			lsum = lsum * corr;
			for (size_t j = 0; j < Bk; j++) {
				const float pj = expf(s[j] - m_new);
				lsum = lsum + pj;
				const float *vj = Vv + (j0 + j) * HL;
				for (size_t d = 0; d < HL; d++)
					o[d] = fmaf(pj, vj[d], o[d]);
			}
			mx = m_new;
		}
		const float inv = 1.0f / lsum;
		for (size_t d = 0; d < HL; d++)
			o[d] = o[d] * inv;
	}
}

/* olmoe_decode / llama_decode (olmoe.c:509-520, llama.c:568-576) of token
 * tok at position pos, then the lm_head product and the greedy pick */
static int lm_decode(struct orc_lm *m, int tok, int pos, float *logits, float *trace_moe_in,
		     uint32_t *trace_ids, float *trace_w, int nthreads)
{
	const size_t E = m->E, NE = m->NE, EI = m->EI, K = m->K, HL = m->HLEN;
	const size_t EQ = m->QH * HL, EK = m->KVH * HL;
	const int olmoe = m->arch == ARCH_OLMOE, te = m->types[0];
	if (m->size >= m->C)
		kv_rotate(m);
	if (pos >= (int)m->C)
		pos = (int)m->size;

	orc_dequant_row((const uint8_t *)m->p[0] + (size_t)tok * qrow_bytes(te, E), te, m->hidden, E);
	for (size_t l = 0; l < m->L; l++) {
		const int *t = m->types + 2 + 6 * l;
		/* the experts' encoding of orc_moe_ffn: gate/up type | down << 8 */
		const int wx = t[4] | (t[5] != t[4] ? t[5] << 8 : 0);
		const size_t gu = EI * qrow_bytes(t[4], E), dn = E * qrow_bytes(t[5], EI);
		const void *const *p = olmoe ? m->p + 3 + 12 * l : m->p + 3 + l * (7 + 3 * NE);
		const void *wq = p[1], *wk = p[2], *wv = p[3], *wo = olmoe ? p[6] : p[4];
		const float *attn_norm = p[0], *ffn_norm = olmoe ? p[7] : p[5];
		const float *router = olmoe ? p[8] : p[6];
		rms_norm_row(m->x, m->hidden, attn_norm, E);
		orc_qmat_mul(m->x, 1, wq, t[0], EQ, E, NULL, 0, m->q);
		orc_qmat_mul(m->x, 1, wk, t[1], EK, E, NULL, 0, m->k);
		orc_qmat_mul(m->x, 1, wv, t[2], EK, E, NULL, 0, m->v);
		if (olmoe) { /* q/k norms over the full vectors (olmoe.c:454-458) */
			rms_norm_row(m->q, m->q, (const float *)p[4], EQ);
			rms_norm_row(m->k, m->k, (const float *)p[5], EK);
		}
		rope(m->q, m->QH, HL, pos, m->theta);
		rope(m->k, m->KVH, HL, pos, m->theta);
		for (size_t kh = 0; kh < m->KVH; kh++) { /* the new row of every kv head */
			memcpy(kv_rows(m, m->kc, l, kh) + m->size * HL, m->k + kh * HL, HL * sizeof(float));
			memcpy(kv_rows(m, m->vc, l, kh) + m->size * HL, m->v + kh * HL, HL * sizeof(float));
		}
		if (olmoe)
			attention_olmoe(m, l);
		else
			attention_llama(m, l);
		orc_qmat_mul(m->attn, 1, wo, t[3], E, EQ, NULL, 0, m->out);
		for (size_t i = 0; i < E; i++) { /* tensor_add (tensor.c:334-353) */
			m->hidden[i] = m->hidden[i] + m->out[i];
			m->resid[i] = m->hidden[i];
		}
		rms_norm_row(m->moe_in, m->hidden, ffn_norm, E);
		if (trace_moe_in)
			memcpy(trace_moe_in + l * E, m->moe_in, E * sizeof(float));
		for (size_t e = 0; e < NE; e++) {
			if (olmoe) { /* tensor_at_q (olmoe.c:20-60) */
				m->ge[e] = (const uint8_t *)p[9] + e * gu;
				m->ue[e] = (const uint8_t *)p[10] + e * gu;
				m->de[e] = (const uint8_t *)p[11] + e * dn;
			} else { /* the per-expert tensors (llama.c:157-166) */
				m->ge[e] = p[7 + e];
				m->ue[e] = p[7 + NE + e];
				m->de[e] = p[7 + 2 * NE + e];
			}
		}
		orc_moe_ffn(m->moe_in, m->out, 1, router, NULL, m->ge, m->ue, m->de, wx, E, EI, NE, K,
			    !olmoe, trace_ids ? trace_ids + l * K : NULL,
			    trace_w ? trace_w + l * K : NULL, NULL, NULL, nthreads);
		for (size_t i = 0; i < E; i++)
			m->hidden[i] = m->resid[i] + m->out[i];
	}
	m->size++;
	rms_norm_row(m->x, m->hidden, (const float *)m->p[2], E);
	float *lg = logits ? logits : malloc(m->V * sizeof(float));
	orc_qmat_mul(m->x, 1, m->p[1], m->types[1], m->V, E, NULL, 0, lg);
	size_t best = 0;
	for (size_t i = 1; i < m->V; i++)
		if (lg[i] > lg[best])
			best = i;
	if (!logits)
		free(lg);
	return (int)best;
}

static void lm_run(struct orc_lm *m, const int *prompt, size_t n_prompt, size_t n_gen,
		   float *logits, int *tokens, int nthreads)
{
	int tok = 0;
	for (size_t i = 0; i < n_prompt; i++)
		tok = lm_decode(m, prompt[i], m->pos++, i + 1 == n_prompt ? logits : NULL, NULL, NULL,
				NULL, nthreads);
	tokens[0] = tok;
	for (size_t s = 1; s <= n_gen; s++) {
		tok = lm_decode(m, tok, m->pos++, logits ? logits + s * m->V : NULL, NULL, NULL, NULL,
				nthreads);
		tokens[s] = tok;
	}
}

orc_olmoe *orc_olmoe_new(size_t layers, size_t E, size_t H, size_t V, size_t NE, size_t topk,
			 size_t EI, size_t C, float theta, int wtype, const void *const *ptrs)
{
	return (orc_olmoe *)lm_new(ARCH_OLMOE, layers, E, H, H, V, NE, topk, EI, C, theta, 0, wtype,
				   NULL, ptrs);
}

orc_olmoe *orc_olmoe_new_typed(size_t layers, size_t E, size_t H, size_t V, size_t NE,
			       size_t topk, size_t EI, size_t C, float theta, const int *types,
			       const void *const *ptrs)
{
	return (orc_olmoe *)lm_new(ARCH_OLMOE, layers, E, H, H, V, NE, topk, EI, C, theta, 0,
				   types[0], types, ptrs);
}

int orc_olmoe_decode(orc_olmoe *m, int tok, int pos, float *logits, float *trace_moe_in,
		     uint32_t *trace_ids, float *trace_w, int nthreads)
{
	return lm_decode(&m->m, tok, pos, logits, trace_moe_in, trace_ids, trace_w, nthreads);
}

void orc_olmoe_run(orc_olmoe *m, const int *prompt, size_t n_prompt, size_t n_gen,
		   float *logits, int *tokens, int nthreads)
{
	lm_run(&m->m, prompt, n_prompt, n_gen, logits, tokens, nthreads);
}

void orc_olmoe_free(orc_olmoe *m)
{
	lm_free(m ? &m->m : NULL);
}

orc_llama *orc_llama_new(size_t layers, size_t E, size_t QH, size_t KVH, size_t V, size_t NE,
			 size_t topk, size_t EI, size_t C, float theta, size_t window, int wtype,
			 const void *const *ptrs)
{
	return (orc_llama *)lm_new(ARCH_LLAMA, layers, E, QH, KVH, V, NE, topk, EI, C, theta, window,
				   wtype, NULL, ptrs);
}

orc_llama *orc_llama_new_typed(size_t layers, size_t E, size_t QH, size_t KVH, size_t V,
			       size_t NE, size_t topk, size_t EI, size_t C, float theta,
			       size_t window, const int *types, const void *const *ptrs)
{
	return (orc_llama *)lm_new(ARCH_LLAMA, layers, E, QH, KVH, V, NE, topk, EI, C, theta, window,
				   types[0], types, ptrs);
}

int orc_llama_decode(orc_llama *m, int tok, int pos, float *logits, float *trace_moe_in,
		     uint32_t *trace_ids, float *trace_w, int nthreads)
{
	return lm_decode(&m->m, tok, pos, logits, trace_moe_in, trace_ids, trace_w, nthreads);
}

void orc_llama_run(orc_llama *m, const int *prompt, size_t n_prompt, size_t n_gen,
		   float *logits, int *tokens, int nthreads)
{
	lm_run(&m->m, prompt, n_prompt, n_gen, logits, tokens, nthreads);
}

void orc_llama_free(orc_llama *m)
{
	lm_free(m ? &m->m : NULL);
}
