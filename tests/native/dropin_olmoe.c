/*
 * TEST: the integration lines of INTEGRATION.md ("OLMoE") around the
 * reference's own OLMoE code.  models/olmoe/olmoe.c is #included from the
 * reference tree at build time (oracle/ref/build_ref.sh, which also links
 * this file against libhip_moe.so); nothing of it is copied.  The lines a
 * maintainer adds live in a field of struct olmoe_layer and at the top of
 * moe_ffn; here they sit in a side table and a wrapper around the static
 * moe_ffn, unchanged otherwise:
 *   - the upload loop of olmoe_load (tensor_at_q views, the HIP_MOE_* types
 *     of the gate/up and down tensors, NULL = stay on the CPU);
 *   - the early return of moe_ffn (hip_moe_ffn, else the CPU body);
 *   - the hip_moe_free loop of olmoe_close.
 * With no GPU the upload returns NULL and the reference's CPU body runs;
 * with one, the layer runs on it.
 */
#include "models/olmoe/olmoe.c"

#include "hip_moe.h"

/* the library's block type of a reference tensor type, 0 = not taken */
static int hip_moe_type(int t)
{
	return t == TENSOR_Q8_0 ? HIP_MOE_Q8_0 : t == TENSOR_Q4_0 ? HIP_MOE_Q4_0 :
	       t == TENSOR_Q4_K ? HIP_MOE_Q4_K : t == TENSOR_Q6_K ? HIP_MOE_Q6_K : 0;
}

/* olmoe_load's loop body for layer i ("At load time") */
static hip_moe_layer *dropin_upload(struct olmoe *model, struct olmoe_layer *hl)
{
	const size_t NE = model->num_experts, E = model->embeddings;
	const size_t EI = model->expert_intermediate;
	const void *g[NE], *u[NE], *d[NE];
	tensor_t v;
	for (size_t e = 0; e < NE; e++) {
		tensor_at_q(hl->gate_exps, e, &v); g[e] = v.qdata;
		tensor_at_q(hl->up_exps, e, &v);   u[e] = v.qdata;
		tensor_at_q(hl->down_exps, e, &v); d[e] = v.qdata;
	}
	const int gt = hip_moe_type(hl->gate_exps->type), dt = hip_moe_type(hl->down_exps->type);
	return gt && dt ? hip_moe_upload_typed(hl->gate_inp->data, g, u, d, gt, dt, E, EI, NE,
					       model->top_k_experts, 0)
			: NULL; /* NULL: this layer stays on the CPU */
}

/* moe_ffn with INTEGRATION.md's early return in front of its body */
static void dropin_moe_ffn(struct olmoe *model, hip_moe_layer *gpu_moe, tensor_t *input,
			   tensor_t *output, size_t l, int *on_gpu)
{
	const size_t T = tensor_len(input);
	if (gpu_moe && hip_moe_ffn(gpu_moe, input->data, output->data, T, NULL, NULL, NULL)) {
		*on_gpu = 1;
		return; /* output[T][E] written; otherwise fall through to the CPU body */
	}
	*on_gpu = 0;
	moe_ffn(model, input, output, l);
}

/*
 * One OLMoE MoE layer through the integration lines: out[T][E].  The stacked
 * *_exps tensors are of reference type wtype & 0xff (gate, up) and
 * wtype >> 8 (down; 0 = the same).  Returns 1 if the GPU took the call, 0 if
 * the CPU body ran; *uploaded says whether the upload returned a layer.
 */
int dropin_olmoe_moe_ffn(const float *x, float *out, size_t T, const float *wr,
			 const void *gate_exps, const void *up_exps, const void *down_exps,
			 int wtype, size_t E, size_t EI, size_t NE, size_t topk, int *uploaded)
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
	const int gtype = wtype & 0xff, dtype = (wtype >> 8) ? (wtype >> 8) : gtype;
	tensor_t *g = tensor_new_mapped((void *)gate_exps, NE * EI * E, gtype);
	tensor_reshape_3d(g, NE, EI, E);
	tensor_t *u = tensor_new_mapped((void *)up_exps, NE * EI * E, gtype);
	tensor_reshape_3d(u, NE, EI, E);
	tensor_t *d = tensor_new_mapped((void *)down_exps, NE * E * EI, dtype);
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

	hip_moe_layer *gpu_moe = dropin_upload(&m, &hl);
	*uploaded = gpu_moe != NULL;
	int on_gpu = 0;
	dropin_moe_ffn(&m, gpu_moe, in, o, 0, &on_gpu);
	hip_moe_free(gpu_moe); /* olmoe_close's loop */

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
	return on_gpu;
}
