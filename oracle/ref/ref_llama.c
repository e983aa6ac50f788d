/*
 * TEST INFRASTRUCTURE: drives the reference's own static moe_ffn of
 * models/llama/llama.c:393-457 (Mixtral: renormalised top-k), compiled from
 * the reference tree (#included at build time by build_ref.sh).
 */
#include "models/llama/llama.c"

void ref_llama_moe_ffn(const float *x, float *out, size_t T, const float *wr,
		       const void *const *gate_e, const void *const *up_e,
		       const void *const *down_e, int wtype, size_t E, size_t EI,
		       size_t NE, size_t topk)
{
	struct llama m;
	struct llama_layer hl;
	memset(&m, 0, sizeof(m));
	memset(&hl, 0, sizeof(hl));
	m.embeddings = E;
	m.expert_intermediate = EI;
	m.num_experts = NE;
	m.top_k_experts = topk;

	tensor_t *gi = tensor_new_mapped((void *)wr, NE * E, TENSOR_F32);
	tensor_reshape_2d(gi, NE, E);
	hl.gate_inp = gi;
	hl.gate_exp = calloc(NE, sizeof(tensor_t *));
	hl.up_exp = calloc(NE, sizeof(tensor_t *));
	hl.down_exp = calloc(NE, sizeof(tensor_t *));
	/* wtype: gate/up type, or'ed with the down type << 8 where it differs */
	const int gt = wtype & 0xff, dt = (wtype >> 8) ? (wtype >> 8) : gt;
	for (size_t e = 0; e < NE; e++) {
		tensor_t *g = tensor_new_mapped((void *)gate_e[e], EI * E, gt);
		tensor_reshape_2d(g, EI, E);
		tensor_t *u = tensor_new_mapped((void *)up_e[e], EI * E, gt);
		tensor_reshape_2d(u, EI, E);
		tensor_t *d = tensor_new_mapped((void *)down_e[e], E * EI, dt);
		tensor_reshape_2d(d, E, EI);
		hl.gate_exp[e] = g;
		hl.up_exp[e] = u;
		hl.down_exp[e] = d;
	}
	m.hl = &hl;

	m.state.gate_logits = tensor_new_zero(2, (size_t)T, (size_t)NE);
	m.state.expert_gate = tensor_new_zero(2, (size_t)1, (size_t)EI);
	m.state.expert_up = tensor_new_zero(2, (size_t)1, (size_t)EI);
	m.state.expert_out = tensor_new_zero(2, (size_t)1, (size_t)E);

	tensor_t *in = tensor_new_mapped((void *)x, T * E, TENSOR_F32);
	tensor_reshape_2d(in, T, E);
	tensor_t *o = tensor_new_mapped(out, T * E, TENSOR_F32);
	tensor_reshape_2d(o, T, E);

	moe_ffn(&m, in, o, 0);

	for (size_t e = 0; e < NE; e++) {
		tensor_free_mapped(hl.gate_exp[e]);
		tensor_free_mapped(hl.up_exp[e]);
		tensor_free_mapped(hl.down_exp[e]);
	}
	free(hl.gate_exp);
	free(hl.up_exp);
	free(hl.down_exp);
	tensor_free(m.state.gate_logits);
	tensor_free(m.state.expert_gate);
	tensor_free(m.state.expert_up);
	tensor_free(m.state.expert_out);
	tensor_free_mapped(gi);
	tensor_free_mapped(in);
	tensor_free_mapped(o);
}

/*
 * The whole model: a struct llama (Mixtral: experts, GQA, optional sliding
 * window) built from caller-held weights, driven through the reference's
 * own llama_prefill / llama_decode (llama.c:564-576) and lm_head product
 * with the greedy pick of main.c:189-193.  ptrs holds 3 + layers * (7 + 3 *
 * NE) pointers: token_embd, output, output_norm, then per layer attn_norm,
 * attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate_inp, the NE gate
 * experts, the NE up experts, the NE down experts.
 */
struct ref_lmodel {
	struct llama m;
	tensor_t **owned;
	size_t n_owned;
};

static const tensor_t *ref_lmap(struct ref_lmodel *r, const void *p, int type, size_t d0,
				size_t d1)
{
	tensor_t *t = tensor_new_mapped((void *)p, d0 * (d1 ? d1 : 1), type);
	if (d1)
		tensor_reshape_2d(t, d0, d1);
	else
		tensor_reshape_1d(t, d0);
	r->owned[r->n_owned++] = t;
	return t;
}

void *ref_llama_model_new_typed(size_t layers, size_t E, size_t QH, size_t KVH, size_t V,
				size_t NE, size_t topk, size_t EI, size_t C, float theta,
				size_t window, const int *types, const void *const *ptrs);

void *ref_llama_model_new(size_t layers, size_t E, size_t QH, size_t KVH, size_t V, size_t NE,
			  size_t topk, size_t EI, size_t C, float theta, size_t window, int wtype,
			  const void *const *ptrs)
{
	int *types = malloc((2 + 6 * layers) * sizeof(int));
	for (size_t i = 0; i < 2 + 6 * layers; i++)
		types[i] = wtype;
	void *r = ref_llama_model_new_typed(layers, E, QH, KVH, V, NE, topk, EI, C, theta, window,
					    types, ptrs);
	free(types);
	return r;
}

/* the same with a block type per tensor (types: token_embd, output, then
 * per layer attn_q, attn_k, attn_v, attn_output, the experts' gate/up, the
 * experts' down) */
void *ref_llama_model_new_typed(size_t layers, size_t E, size_t QH, size_t KVH, size_t V,
				size_t NE, size_t topk, size_t EI, size_t C, float theta,
				size_t window, const int *types, const void *const *ptrs)
{
	struct ref_lmodel *r = calloc(1, sizeof(*r));
	struct llama *m = &r->m;
	r->owned = calloc(3 + layers * (7 + 3 * NE), sizeof(tensor_t *));
	m->context = C;
	m->embeddings = E;
	m->q_heads = QH;
	m->kv_heads = KVH;
	m->layers = layers;
	m->head_len = E / QH;
	m->vocab_len = V;
	m->num_experts = NE;
	m->top_k_experts = topk;
	m->expert_intermediate = EI;
	m->rope_theta = theta;
	m->sliding_window = window;
	m->bos_id = 0;
	m->eos_id = -1;
	m->tool_calls_token = -1;
	m->hlen_sq = sqrt((scalar_t)m->head_len);
	const size_t HLEN = m->head_len;

	m->wte = ref_lmap(r, ptrs[0], types[0], V, E);
	m->lm_head = ref_lmap(r, ptrs[1], types[1], V, E);
	m->output_norm = ref_lmap(r, ptrs[2], TENSOR_F32, E, 0);
	m->hl = calloc(layers, sizeof(*m->hl));
	for (size_t l = 0; l < layers; l++) {
		const void *const *p = ptrs + 3 + l * (7 + 3 * NE);
		const int *t = types + 2 + 6 * l;
		struct llama_layer *hl = &m->hl[l];
		hl->attn_norm = ref_lmap(r, p[0], TENSOR_F32, E, 0);
		hl->q_weight = ref_lmap(r, p[1], t[0], QH * HLEN, E);
		hl->k_weight = ref_lmap(r, p[2], t[1], KVH * HLEN, E);
		hl->v_weight = ref_lmap(r, p[3], t[2], KVH * HLEN, E);
		hl->o_weight = ref_lmap(r, p[4], t[3], E, QH * HLEN);
		hl->ffn_norm = ref_lmap(r, p[5], TENSOR_F32, E, 0);
		hl->gate_inp = ref_lmap(r, p[6], TENSOR_F32, NE, E);
		hl->gate_exp = calloc(NE, sizeof(tensor_t *));
		hl->up_exp = calloc(NE, sizeof(tensor_t *));
		hl->down_exp = calloc(NE, sizeof(tensor_t *));
		for (size_t e = 0; e < NE; e++) {
			hl->gate_exp[e] = ref_lmap(r, p[7 + e], t[4], EI, E);
			hl->up_exp[e] = ref_lmap(r, p[7 + NE + e], t[4], EI, E);
			hl->down_exp[e] = ref_lmap(r, p[7 + 2 * NE + e], t[5], E, EI);
		}
	}
	/* llama_load's state tensors (llama.c:177-200) and cache */
	m->state.output = tensor_new_zero(2, C, E);
	m->state.hidden = tensor_new_zero(2, C, E);
	m->state.q = tensor_new_zero(2, C, QH * HLEN);
	m->state.k = tensor_new_zero(2, C, KVH * HLEN);
	m->state.v = tensor_new_zero(2, C, KVH * HLEN);
	m->state.qh = tensor_new_zero(2, C, HLEN);
	m->state.masked_attn = tensor_new_zero(2, C, C);
	m->state.attn = tensor_new_zero(2, C, E);
	m->state.attn_residual = tensor_new_zero(2, C, E);
	m->state.gate_logits = tensor_new_zero(2, C, NE);
	m->state.expert_gate = tensor_new_zero(2, 1, EI);
	m->state.expert_up = tensor_new_zero(2, 1, EI);
	m->state.expert_out = tensor_new_zero(2, 1, E);
	m->state.moe_out = tensor_new_zero(2, C, E);
	m->state.logits = tensor_new_zero(1, V);
	m->cache = kvcache_alloc(layers, C, KVH, HLEN);
	m->cache->sliding_window = window;
	return r;
}

static int ref_lpick(struct llama *m, size_t row, float *logits_out)
{
	tensor_t last_row;
	tensor_at(m->state.output, row, &last_row);
	tensor_reshape_2d(&last_row, 1, m->embeddings);
	tensor_mma_transposed_2x2(m->state.logits, &last_row, m->lm_head, NULL);
	tensor_reshape_1d(m->state.logits, m->vocab_len);
	if (logits_out)
		memcpy(logits_out, m->state.logits->data, m->vocab_len * sizeof(float));
	size_t token = 0; /* main.c:189-193 */
	for (size_t i = 1; i < m->state.logits->totlen; i++)
		if (m->state.logits->data[i] > m->state.logits->data[token])
			token = i;
	return (int)token;
}

/* llama_generate (llama.c:578-667) without tokenizer, tools and EOS stop,
 * as ref_olmoe_model_run: prompt (one llama_prefill, or one llama_decode
 * per id), then n_gen greedy llama_decode steps */
void ref_llama_model_run(void *h, const int *prompt, size_t n_prompt, int prefill, size_t n_gen,
			 float *logits, int *tokens)
{
	struct ref_lmodel *r = h;
	struct llama *m = &r->m;
	const size_t V = m->vocab_len;
	int *toks = malloc(n_prompt * sizeof(int)), *poss = malloc(n_prompt * sizeof(int));
	for (size_t i = 0; i < n_prompt; i++) {
		toks[i] = prompt[i];
		poss[i] = m->pos + (int)i;
	}
	int tok;
	if (prefill) {
		llama_prefill(m, toks, poss, n_prompt, m->state.output);
		m->pos += (int)n_prompt;
		tok = ref_lpick(m, n_prompt - 1, logits);
	} else {
		for (size_t i = 0; i < n_prompt; i++) {
			llama_decode(m, toks[i], m->pos, m->state.output);
			m->pos++;
		}
		tok = ref_lpick(m, 0, logits);
	}
	tokens[0] = tok;
	for (size_t s = 1; s <= n_gen; s++) {
		llama_decode(m, tok, m->pos, m->state.output);
		m->pos++;
		tok = ref_lpick(m, 0, logits ? logits + s * V : NULL);
		tokens[s] = tok;
	}
	free(toks);
	free(poss);
}

void ref_llama_model_free(void *h)
{
	struct ref_lmodel *r = h;
	struct llama *m = &r->m;
	for (size_t i = 0; i < r->n_owned; i++)
		tensor_free_mapped(r->owned[i]);
	free(r->owned);
	for (size_t l = 0; l < m->layers; l++) {
		free(m->hl[l].gate_exp);
		free(m->hl[l].up_exp);
		free(m->hl[l].down_exp);
	}
	free(m->hl);
	tensor_free(m->state.output);
	tensor_free(m->state.hidden);
	tensor_free(m->state.q);
	tensor_free(m->state.k);
	tensor_free(m->state.v);
	tensor_free(m->state.qh);
	tensor_free(m->state.masked_attn);
	tensor_free(m->state.attn);
	tensor_free(m->state.attn_residual);
	tensor_free(m->state.gate_logits);
	tensor_free(m->state.expert_gate);
	tensor_free(m->state.expert_up);
	tensor_free(m->state.expert_out);
	tensor_free(m->state.moe_out);
	tensor_free(m->state.logits);
	kvcache_free(m->cache);
	free(r);
}
