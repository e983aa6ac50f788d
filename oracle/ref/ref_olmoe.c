/*
 * TEST INFRASTRUCTURE: drives the reference's own static moe_ffn of
 * models/olmoe/olmoe.c:343-407, compiled from the reference tree (the file is
 * #included from there at build time, see build_ref.sh; nothing is copied).
 * Used to produce golden vectors for the oracle.
 */
#include "models/olmoe/olmoe.c"

void ref_olmoe_moe_ffn(const float *x, float *out, size_t T, const float *wr,
		       const void *gate_exps, const void *up_exps, const void *down_exps,
		       int wtype, size_t E, size_t EI, size_t NE, size_t topk)
{
	struct olmoe m;
	struct olmoe_layer hl;
	memset(&m, 0, sizeof(m));
	memset(&hl, 0, sizeof(hl));
	m.embeddings = E;
	m.expert_intermediate = EI;
	m.num_experts = NE;
	m.top_k_experts = topk;

	tensor_t *gi = tensor_new_mapped((void *)wr, NE * E, TENSOR_F32);
	tensor_reshape_2d(gi, NE, E);
	/* wtype: gate/up type, or'ed with the down type << 8 where it differs */
	const int gt = wtype & 0xff, dt = (wtype >> 8) ? (wtype >> 8) : gt;
	tensor_t *g = tensor_new_mapped((void *)gate_exps, NE * EI * E, gt);
	tensor_reshape_3d(g, NE, EI, E);
	tensor_t *u = tensor_new_mapped((void *)up_exps, NE * EI * E, gt);
	tensor_reshape_3d(u, NE, EI, E);
	tensor_t *d = tensor_new_mapped((void *)down_exps, NE * E * EI, dt);
	tensor_reshape_3d(d, NE, E, EI);
	hl.gate_inp = gi;
	hl.gate_exps = g;
	hl.up_exps = u;
	hl.down_exps = d;
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

	tensor_free(m.state.gate_logits);
	tensor_free(m.state.expert_gate);
	tensor_free(m.state.expert_up);
	tensor_free(m.state.expert_out);
	tensor_free_mapped(gi);
	tensor_free_mapped(g);
	tensor_free_mapped(u);
	tensor_free_mapped(d);
	tensor_free_mapped(in);
	tensor_free_mapped(o);
}

/*
 * The whole model: a struct olmoe built from caller-held weights (no GGUF),
 * driven through the reference's own olmoe_prefill / olmoe_decode
 * (olmoe.c:502-520) and lm_head product (olmoe.c:560-580) with the greedy
 * pick of main.c:189-193 (first maximum wins).  ptrs holds 3 + 12 * layers
 * pointers: token_embd, output, output_norm, then per layer attn_norm,
 * attn_q, attn_k, attn_v, attn_q_norm, attn_k_norm, attn_output, ffn_norm,
 * ffn_gate_inp, ffn_gate_exps, ffn_up_exps, ffn_down_exps.  Quantized
 * tensors are wtype blocks, norms and the router fp32.
 */
struct ref_model {
	struct olmoe m;
	tensor_t **owned;
	size_t n_owned;
};

static const tensor_t *ref_map(struct ref_model *r, const void *p, int type, size_t d0,
			       size_t d1, size_t d2)
{
	size_t n = d0 * (d1 ? d1 : 1) * (d2 ? d2 : 1);
	tensor_t *t = tensor_new_mapped((void *)p, n, type);
	if (d2)
		tensor_reshape_3d(t, d0, d1, d2);
	else if (d1)
		tensor_reshape_2d(t, d0, d1);
	else
		tensor_reshape_1d(t, d0);
	r->owned[r->n_owned++] = t;
	return t;
}

void *ref_olmoe_model_new_typed(size_t layers, size_t E, size_t H, size_t V, size_t NE,
				size_t topk, size_t EI, size_t C, float theta, const int *types,
				const void *const *ptrs);

void *ref_olmoe_model_new(size_t layers, size_t E, size_t H, size_t V, size_t NE, size_t topk,
			  size_t EI, size_t C, float theta, int wtype, const void *const *ptrs)
{
	int *types = malloc((2 + 6 * layers) * sizeof(int));
	for (size_t i = 0; i < 2 + 6 * layers; i++)
		types[i] = wtype;
	void *r = ref_olmoe_model_new_typed(layers, E, H, V, NE, topk, EI, C, theta, types, ptrs);
	free(types);
	return r;
}

/* the same with a block type per tensor, as a GGUF's tensors carry them:
 * types[0] token_embd, types[1] output, then per layer attn_q, attn_k,
 * attn_v, attn_output, ffn_gate/up_exps, ffn_down_exps */
void *ref_olmoe_model_new_typed(size_t layers, size_t E, size_t H, size_t V, size_t NE,
				size_t topk, size_t EI, size_t C, float theta, const int *types,
				const void *const *ptrs)
{
	struct ref_model *r = calloc(1, sizeof(*r));
	struct olmoe *m = &r->m;
	r->owned = calloc(3 + 12 * layers, sizeof(tensor_t *));
	m->context = C;
	m->embeddings = E;
	m->heads = H;
	m->layers = layers;
	m->head_len = E / H;
	m->vocab_len = V;
	m->num_experts = NE;
	m->top_k_experts = topk;
	m->expert_intermediate = EI;
	m->rope_theta = theta;
	m->bos_id = 0;
	m->eos_id = -1;
	m->hlen_sq = sqrt((scalar_t)m->head_len);
	size_t HLEN = m->head_len;

	m->wte = ref_map(r, ptrs[0], types[0], V, E, 0);
	m->lm_head = ref_map(r, ptrs[1], types[1], V, E, 0);
	m->output_norm = ref_map(r, ptrs[2], TENSOR_F32, E, 0, 0);
	m->hl = calloc(layers, sizeof(*m->hl));
	for (size_t l = 0; l < layers; l++) {
		const void *const *p = ptrs + 3 + 12 * l;
		const int *t = types + 2 + 6 * l;
		m->hl[l].attn_norm = ref_map(r, p[0], TENSOR_F32, E, 0, 0);
		m->hl[l].q_weight = ref_map(r, p[1], t[0], E, E, 0);
		m->hl[l].k_weight = ref_map(r, p[2], t[1], E, E, 0);
		m->hl[l].v_weight = ref_map(r, p[3], t[2], E, E, 0);
		m->hl[l].q_norm = ref_map(r, p[4], TENSOR_F32, E, 0, 0);
		m->hl[l].k_norm = ref_map(r, p[5], TENSOR_F32, E, 0, 0);
		m->hl[l].o_weight = ref_map(r, p[6], t[3], E, E, 0);
		m->hl[l].ffn_norm = ref_map(r, p[7], TENSOR_F32, E, 0, 0);
		m->hl[l].gate_inp = ref_map(r, p[8], TENSOR_F32, NE, E, 0);
		m->hl[l].gate_exps = ref_map(r, p[9], t[4], NE, EI, E);
		m->hl[l].up_exps = ref_map(r, p[10], t[4], NE, EI, E);
		m->hl[l].down_exps = ref_map(r, p[11], t[5], NE, E, EI);
	}
	/* olmoe_load's state tensors (olmoe.c:185-199) and cache */
	m->state.output = tensor_new_zero(2, C, E);
	m->state.hidden = tensor_new_zero(2, C, E);
	m->state.q = tensor_new_zero(2, C, E);
	m->state.k = tensor_new_zero(2, C, E);
	m->state.v = tensor_new_zero(2, C, E);
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
	m->cache = kvcache_alloc(layers, C, H, HLEN);
	return r;
}

/* main.c:189-193 */
static int ref_argmax(const tensor_t *logits)
{
	size_t token = 0;
	for (size_t i = 1; i < logits->totlen; i++)
		if (logits->data[i] > logits->data[token])
			token = i;
	return (int)token;
}

/* olmoe_generate's lm_head step (olmoe.c:558-564): logits of output row `row` */
static int ref_pick(struct olmoe *m, size_t row, float *logits_out)
{
	tensor_t last_row;
	tensor_at(m->state.output, row, &last_row);
	tensor_reshape_2d(&last_row, 1, m->embeddings);
	tensor_mma_transposed_2x2(m->state.logits, &last_row, m->lm_head, NULL);
	tensor_reshape_1d(m->state.logits, m->vocab_len);
	if (logits_out)
		memcpy(logits_out, m->state.logits->data, m->vocab_len * sizeof(float));
	return ref_argmax(m->state.logits);
}

/*
 * olmoe_generate (olmoe.c:522-600) without the tokenizer and without the EOS
 * stop: the prompt ids go in as given (prefill = 1: one olmoe_prefill, as
 * generate does; 0: one olmoe_decode per prompt id), then n_gen greedy
 * olmoe_decode steps.  tokens[0..n_gen] are the n_gen + 1 picks, logits
 * (optional) their [n_gen + 1][V] logits.  Continues from the model's
 * current position (model->pos), like generate.
 */
void ref_olmoe_model_run(void *h, const int *prompt, size_t n_prompt, int prefill, size_t n_gen,
			 float *logits, int *tokens)
{
	struct ref_model *r = h;
	struct olmoe *m = &r->m;
	const size_t V = m->vocab_len;
	int *toks = malloc(n_prompt * sizeof(int)), *poss = malloc(n_prompt * sizeof(int));
	for (size_t i = 0; i < n_prompt; i++) {
		toks[i] = prompt[i];
		poss[i] = m->pos + (int)i;
	}
	int tok;
	if (prefill) {
		olmoe_prefill(m, toks, poss, n_prompt, m->state.output);
		m->pos += (int)n_prompt;
		tok = ref_pick(m, n_prompt - 1, logits);
	} else {
		for (size_t i = 0; i < n_prompt; i++) {
			olmoe_decode(m, toks[i], m->pos, m->state.output);
			m->pos++;
		}
		tok = ref_pick(m, 0, logits);
	}
	tokens[0] = tok;
	for (size_t s = 1; s <= n_gen; s++) {
		olmoe_decode(m, tok, m->pos, m->state.output);
		m->pos++;
		tok = ref_pick(m, 0, logits ? logits + s * V : NULL);
		tokens[s] = tok;
	}
	free(toks);
	free(poss);
}

void ref_olmoe_model_free(void *h)
{
	struct ref_model *r = h;
	struct olmoe *m = &r->m;
	for (size_t i = 0; i < r->n_owned; i++)
		tensor_free_mapped(r->owned[i]);
	free(r->owned);
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
