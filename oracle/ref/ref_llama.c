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
	for (size_t e = 0; e < NE; e++) {
		tensor_t *g = tensor_new_mapped((void *)gate_e[e], EI * E, wtype);
		tensor_reshape_2d(g, EI, E);
		tensor_t *u = tensor_new_mapped((void *)up_e[e], EI * E, wtype);
		tensor_reshape_2d(u, EI, E);
		tensor_t *d = tensor_new_mapped((void *)down_e[e], E * EI, wtype);
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
