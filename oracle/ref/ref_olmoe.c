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
	tensor_t *g = tensor_new_mapped((void *)gate_exps, NE * EI * E, wtype);
	tensor_reshape_3d(g, NE, EI, E);
	tensor_t *u = tensor_new_mapped((void *)up_exps, NE * EI * E, wtype);
	tensor_reshape_3d(u, NE, EI, E);
	tensor_t *d = tensor_new_mapped((void *)down_exps, NE * E * EI, wtype);
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
