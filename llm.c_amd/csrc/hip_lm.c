/*
 * hip_lm.c - host layer of the whole-model decode (include/hip_lm.h).
 *
 * Owns the device copies of every tensor, the fp32 KV cache, the step's
 * buffers and a small device state block (token, position, cache row), and
 * enqueues one decode step as
 *   embed -> per layer [rmsnorm -> qkv product -> q/k norm + RoPE + cache
 *   row -> attention -> output product + residual -> rmsnorm -> MoE layer]
 *   -> residual + final rmsnorm -> lm_head product -> greedy pick
 * (olmoe_forward for one token, olmoe.c:409-500, then olmoe.c:558-564 and
 * main.c:189-193).  The residual adds ride on other steps: the output
 * product's `add` operand is the residual stream, and the MoE output is
 * added to it in front of the next RMSNorm.  Every step kernel reads its
 * counters from the device, so generate captures a step once per shape
 * (with and without the lm_head) and replays it.
 */
#include "hip_lm.h"
#include "lm_internal.h"
#include "moe_internal.h"
#include "moe_synth.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* rows of one prefill launch group of a lockstep batch's prompts */
#define PF_GROUP_ROWS 2048

struct lm_layer {
	float *attn_norm, *q_norm, *k_norm, *ffn_norm;
	uint8_t *wqkv; /* [q rows | k rows | v rows][E] blocks (one block type) */
	uint8_t *wo;   /* [E][heads * 128] blocks */
	hip_moe_layer *moe;
	/* mixed block types (the generic step): each tensor's type and its
	 * product's workgroups.  The first nqkv of q, k, v (those sharing q's
	 * type, in that order) are stacked in wq and run as one product
	 * (their rows are consecutive in the step's q/k/v row); wk and wv are
	 * set only for tensors not stacked */
	uint8_t *wq, *wk, *wv;
	int tq, tk, tv, to;
	int gq, gk, gv, go;
	int nqkv;
};

struct hip_lm {
	int arch, wtype, device;
	/* generic: the matrices are not all Q8_0 or all Q4_0 (per-tensor types,
	 * K-quants): the step runs separate norm, product and attention
	 * launches instead of the fused step kernels */
	int generic, embd_type, output_type, ghead;
	float *d_x; /* generic step: the normalised row a product takes */
	size_t L, E, H, KH, HL, V, C, NE, K, EI, window;
	float theta, scale; /* attention: scores / scale (OLMoE) or * scale (Mixtral) */
	size_t EQ, EKV; /* rows of q, and of k (= of v) */
	size_t weight_bytes;
	hipStream_t stream;

	uint8_t *d_wte, *d_head;
	float *d_onorm;
	struct lm_layer *ly;
	int grid_qkv, grid_o, grid_head; /* resident workgroups of the one-token products */

	float *d_kc, *d_vc; /* [L][KH][C][HL] */
	float *d_freq;      /* [HL / 2] rope frequencies */
	float *d_h0, *d_h1, *d_qkv, *d_attn, *d_moe_in, *d_moe_out, *d_logits;
	uint64_t *d_part;   /* tagged attention partials [H][chunks][HL + 2] */
	uint64_t *d_rows_t; /* tagged output-product rows [E] */
	uint64_t *d_best;   /* tagged per-workgroup maxima of the lm_head [2 * grid] */
	uint32_t *d_cnt;    /* attention arrival counters [H] */
	uint32_t *d_ids;   /* [L][K] */
	float *d_w;        /* [L][K] */
	LmState *d_st;
	int *d_prompt, *d_tokens;
	size_t prompt_cap, tokens_cap;

	/* host mirror of the counters */
	LmState st;
	/* captured steps without / with the lm_head, one per count of active
	 * attention chunks (the attention grid), captured when first needed */
	int nch;
	hipGraphExec_t *g_body, *g_head;
	unsigned graph_gen; /* the MoE layers' scratch generation the graphs name */
	unsigned path_gen;  /* forced MoE path changes (hip_lm_set_moe_path) */
	hipEvent_t ev0, ev1;

	/* prefill: a prompt of up to pf_cap rows in one forward, rows [T][.] */
	size_t pf_cap, pf_heads; /* rows, and sequences whose last rows take the lm_head */
	float *d_pf_h0, *d_pf_h1, *d_pf_x, *d_pf_qkv, *d_pf_q, *d_pf_attn, *d_pf_min,
		*d_pf_mout;
	void *d_pf_split; /* the matrix-core products' partial sums */
	LmState *d_pst;   /* step 0 of one-id prompts: row s takes prompt[s] */
};

static void lm_err(const char *fmt, ...)
{
	char buf[512];
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(buf, sizeof(buf), fmt, ap);
	va_end(ap);
	moe_set_error(buf);
}

#define HIPCHK(call, what)                                                        \
	do {                                                                      \
		hipError_t e_ = (call);                                           \
		if (e_ != hipSuccess) {                                           \
			lm_err("%s: %s", what, hipGetErrorString(e_));             \
			goto fail;                                                \
		}                                                                 \
	} while (0)

#define LCHK(rc, what)                                                            \
	do {                                                                      \
		int r_ = (rc);                                                    \
		if (r_ != 0) {                                                    \
			lm_err("%s: %s", what, hipGetErrorString((hipError_t)r_));  \
			return 0;                                                 \
		}                                                                 \
	} while (0)

static size_t qbytes(int wtype, size_t rows, size_t cols)
{
	return rows * (cols / 32) * (wtype == HIP_MOE_Q8_0 ? 34 : 18);
}

static int is_kq(int t)
{
	return t == HIP_MOE_Q4_K || t == HIP_MOE_Q6_K;
}

/* tensor i (0 attn_q, 1 attn_k, 2 attn_v, 3 attn_output, 4 experts' gate/up,
 * 5 experts' down) of layer l */
static int layer_type(const hip_lm_desc *d, size_t l, int i)
{
	const int t = d->layer_types ? d->layer_types[6 * l + i] : 0;
	return t ? t : d->wtype;
}

/* bytes of a rows x cols matrix in type t, with the K-quant products'
 * read slack past the end */
static size_t tbytes(int t, size_t rows, size_t cols)
{
	return rows * moe_row_bytes(t, cols) + (is_kq(t) ? MOE_KQ_SLACK : 0);
}

static int upload(void **dst, const void *src, size_t bytes, const char *what)
{
	HIPCHK(hipMalloc(dst, bytes), what);
	HIPCHK(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice), what);
	return 1;
fail:
	return 0;
}

/* a rows x cols matrix of type t (tbytes: the K-quant read slack after it,
 * zeroed) */
static int upload_t(uint8_t **dst, const void *src, int t, size_t rows, size_t cols,
		    const char *what)
{
	const size_t n = rows * moe_row_bytes(t, cols), all = tbytes(t, rows, cols);
	HIPCHK(hipMalloc((void **)dst, all), what);
	if (all > n)
		HIPCHK(hipMemset(*dst + n, 0, all - n), what);
	HIPCHK(hipMemcpy(*dst, src, n, hipMemcpyHostToDevice), what);
	return 1;
fail:
	return 0;
}

/* n matrices of one type t and `cols` columns, rows[i] rows each, stacked
 * into one buffer (the rows of matrix i after those of matrix i - 1) */
static int upload_stacked(uint8_t **dst, const void *const *src, const size_t *rows, int n,
			  int t, size_t cols, const char *what)
{
	const size_t rb = moe_row_bytes(t, cols);
	size_t all = 0, off = 0;
	for (int i = 0; i < n; i++)
		all += rows[i];
	const size_t n_bytes = all * rb, bytes = tbytes(t, all, cols);
	HIPCHK(hipMalloc((void **)dst, bytes), what);
	if (bytes > n_bytes)
		HIPCHK(hipMemset(*dst + n_bytes, 0, bytes - n_bytes), what);
	for (int i = 0; i < n; i++) {
		HIPCHK(hipMemcpy(*dst + off, src[i], rows[i] * rb, hipMemcpyHostToDevice), what);
		off += rows[i] * rb;
	}
	return 1;
fail:
	return 0;
}

static void drop_graphs(hip_lm *M)
{
	for (int i = 0; M->g_body && i <= M->nch; i++) {
		if (M->g_body[i])
			hipGraphExecDestroy(M->g_body[i]);
		if (M->g_head[i])
			hipGraphExecDestroy(M->g_head[i]);
		M->g_body[i] = M->g_head[i] = NULL;
	}
}

/* the sum of the MoE layers' scratch generations: it changes whenever a
 * layer reallocates its scratch (a lockstep batch reserving more tokens),
 * after which step graphs captured before name freed buffers */
static unsigned moe_gen(const hip_lm *M)
{
	unsigned g = M->path_gen * 1000003u; /* a forced path changes the launches */
	for (size_t l = 0; M->ly && l < M->L; l++)
		g += moe_scratch_gen(M->ly[l].moe);
	return g;
}

static void free_prefill(hip_lm *M)
{
	void *bufs[] = {M->d_pf_h0,   M->d_pf_h1,  M->d_pf_x,    M->d_pf_qkv, M->d_pf_q,
			M->d_pf_attn, M->d_pf_min, M->d_pf_mout, M->d_pf_split};
	for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
		hipFree(bufs[i]);
	M->d_pf_h0 = M->d_pf_h1 = M->d_pf_x = M->d_pf_qkv = M->d_pf_q = M->d_pf_attn = NULL;
	M->d_pf_min = M->d_pf_mout = NULL;
	M->d_pf_split = NULL;
	M->pf_cap = 0;
	M->pf_heads = 0;
}

void hip_lm_free(hip_lm *M)
{
	if (!M)
		return;
	drop_graphs(M);
	free_prefill(M);
	hipFree(M->d_pst);
	free(M->g_body);
	free(M->g_head);
	if (M->ly) {
		for (size_t l = 0; l < M->L; l++) {
			struct lm_layer *y = &M->ly[l];
			hipFree(y->attn_norm);
			hipFree(y->q_norm);
			hipFree(y->k_norm);
			hipFree(y->ffn_norm);
			hipFree(y->wqkv);
			hipFree(y->wo);
			hipFree(y->wq);
			hipFree(y->wk);
			hipFree(y->wv);
			hip_moe_free(y->moe);
		}
		free(M->ly);
	}
	hipFree(M->d_x);
	void *bufs[] = {M->d_wte, M->d_head, M->d_onorm, M->d_kc, M->d_vc, M->d_freq, M->d_h0,
			M->d_h1, M->d_qkv, M->d_attn, M->d_moe_in, M->d_moe_out, M->d_part,
			M->d_rows_t, M->d_best, M->d_cnt, M->d_logits, M->d_ids, M->d_w,
			M->d_st, M->d_prompt, M->d_tokens};
	for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
		hipFree(bufs[i]);
	if (M->ev0)
		hipEventDestroy(M->ev0);
	if (M->ev1)
		hipEventDestroy(M->ev1);
	if (M->stream)
		hipStreamDestroy(M->stream);
	free(M);
}

static int type_ok(int t)
{
	return t == HIP_MOE_Q8_0 || t == HIP_MOE_Q4_0 || t == HIP_MOE_Q4_K || t == HIP_MOE_Q6_K;
}

/* a product over K columns in type t runs for one token */
static int product_ok(int t, size_t K)
{
	if (is_kq(t))
		return moe_kq_supported(t, (int)K);
	return K % 64 == 0 && K / 64 >= 4 && K / 64 <= 64 && ((K / 64) & (K / 64 - 1)) == 0;
}

static int product_grid(int t, size_t K)
{
	return is_kq(t) ? moe_kq_grid(t, (int)K, 1) : moe_qgemv_grid(t, (int)K, 1);
}

/* out[N] = add + x . W^T for one token (add NULL or [N]) in type t */
static int vec_product(int t, const uint8_t *W, int N, int K, const float *x, const float *add,
		       float *out, int grid, hipStream_t s)
{
	if (is_kq(t))
		LCHK(moe_launch_kq_gemv(t, W, N, K, x, 1, add, 0, out, grid, s), "product");
	else
		LCHK(moe_launch_qgemv(t, W, N, K, x, 1, add, 0, out, grid, s), "product");
	return 1;
}

static int check_desc(const hip_lm_desc *d)
{
	if (!d) {
		lm_err("lm_upload: NULL descriptor");
		return 0;
	}
	if (d->arch != HIP_LM_OLMOE && d->arch != HIP_LM_MIXTRAL) {
		lm_err("lm_upload: unknown arch %d", d->arch);
		return 0;
	}
	if (!type_ok(d->wtype)) {
		lm_err("lm_upload: unsupported weight type %d", d->wtype);
		return 0;
	}
	if ((d->embd_type && !type_ok(d->embd_type)) ||
	    (d->output_type && !type_ok(d->output_type))) {
		lm_err("lm_upload: unsupported embedding / output type %d / %d", d->embd_type,
		       d->output_type);
		return 0;
	}
	for (size_t i = 0; d->layer_types && i < 6 * d->layers; i++)
		if (d->layer_types[i] && !type_ok(d->layer_types[i])) {
			lm_err("lm_upload: unsupported type %d of layer %zu", d->layer_types[i], i / 6);
			return 0;
		}
	if (!d->layers || !d->E || !d->heads || !d->kv_heads || d->heads % d->kv_heads ||
	    !d->vocab || d->vocab > 0x7fffffff || d->context < 2 || d->context > (1u << 24)) {
		lm_err("lm_upload: bad sizes (layers %zu, E %zu, heads %zu/%zu, vocab %zu, "
		       "context %zu)", d->layers, d->E, d->heads, d->kv_heads, d->vocab, d->context);
		return 0;
	}
	if (d->layers >= LM_HEAD_SLOT) {
		lm_err("lm_upload: at most %d layers", LM_HEAD_SLOT - 1);
		return 0;
	}
	if (lm_attn_chunks((int)d->context, (int)d->sliding_window) > LM_MAX_CHUNKS) {
		lm_err("lm_upload: context %zu (window %zu) beyond %d attention chunks",
		       d->context, d->sliding_window, LM_MAX_CHUNKS);
		return 0;
	}
	if (d->arch == HIP_LM_OLMOE && d->heads * LM_HLEN != d->E) {
		lm_err("lm_upload: OLMoE needs heads * %d == E", LM_HLEN);
		return 0;
	}
	if (!d->token_embd || !d->output || !d->output_norm || !d->attn_norm || !d->attn_q ||
	    !d->attn_k || !d->attn_v || !d->attn_o || !d->ffn_norm || !d->gate_inp ||
	    !d->gate_e || !d->up_e || !d->down_e ||
	    (d->arch == HIP_LM_OLMOE && (!d->q_norm || !d->k_norm))) {
		lm_err("lm_upload: NULL tensor pointer");
		return 0;
	}
	return 1;
}

hip_lm *hip_lm_upload(const hip_lm_desc *d)
{
	hip_lm *M = NULL;
	uint8_t *stage = NULL;
	int ndev = 0;
	if (!check_desc(d))
		return NULL;
	if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
		lm_err("lm_upload: no HIP device");
		return NULL;
	}
	M = calloc(1, sizeof(*M));
	if (!M) {
		lm_err("lm_upload: out of host memory");
		return NULL;
	}
	M->arch = d->arch;
	M->wtype = d->wtype;
	M->L = d->layers;
	M->E = d->E;
	M->H = d->heads;
	M->KH = d->kv_heads;
	M->HL = LM_HLEN;
	M->V = d->vocab;
	M->C = d->context;
	M->NE = d->NE;
	M->K = d->topk;
	M->EI = d->EI;
	M->window = d->sliding_window;
	M->theta = d->rope_theta;
	M->embd_type = d->embd_type ? d->embd_type : d->wtype;
	M->output_type = d->output_type ? d->output_type : d->wtype;
	M->generic = (d->wtype != HIP_MOE_Q8_0 && d->wtype != HIP_MOE_Q4_0) ||
		     M->embd_type != d->wtype || M->output_type != d->wtype;
	for (size_t l = 0; l < M->L; l++)
		for (int i = 0; i < 6; i++)
			M->generic |= layer_type(d, l, i) != d->wtype;
	/* hlen_sq = sqrt((scalar_t)HLEN) (olmoe.c:150, llama.c:118): OLMoE
	 * divides the scores by it, Mixtral's flash_attention multiplies them
	 * by 1.0f / hlen_sq (llama.c:324) */
	{
		const float hlen_sq = (float)sqrt((double)(float)M->HL);
		M->scale = d->arch == HIP_LM_OLMOE ? hlen_sq : 1.0f / hlen_sq;
	}
	M->EQ = M->H * M->HL;
	M->EKV = M->KH * M->HL;
	M->nch = lm_attn_chunks((int)M->C, (int)M->window);
	M->g_body = calloc((size_t)M->nch + 1, sizeof(hipGraphExec_t));
	M->g_head = calloc((size_t)M->nch + 1, sizeof(hipGraphExec_t));
	if (!M->g_body || !M->g_head) {
		lm_err("lm_upload: out of host memory");
		goto fail;
	}
	const int wt = d->wtype;
	const size_t E = M->E;

	HIPCHK(hipGetDevice(&M->device), "hipGetDevice");
	HIPCHK(hipStreamCreateWithFlags(&M->stream, hipStreamNonBlocking), "hipStreamCreate");
	HIPCHK(hipEventCreate(&M->ev0), "hipEventCreate");
	HIPCHK(hipEventCreate(&M->ev1), "hipEventCreate");

	if (!M->generic) {
		/* products: one token, K = E (qkv) and heads * 128 (output); the
		 * workgroups resident at once, queried here, not under capture */
		M->grid_qkv = lm_gemv_grid(0, wt, (int)E, (int)(M->EQ + 2 * M->EKV));
		M->grid_o = lm_gemv_grid(1, wt, (int)M->EQ, (int)E);
		M->grid_head = lm_gemv_grid(2, wt, (int)E, (int)M->V);
		/* (the output product's last workgroup gathers E rows in the LDS
		 * that staged its heads * 128 inputs) */
		if (M->grid_qkv <= 0 || M->grid_o <= 0 || M->grid_head <= 0 ||
		    M->grid_head > LM_MAX_HEAD_WG || M->grid_o > LM_MAX_HEAD_WG ||
		    E * 64 > M->EQ * 68) {
			lm_err("lm_upload: E=%zu / heads*128=%zu not supported by the dense product",
			       E, M->EQ);
			goto fail;
		}
	} else {
		M->ghead = product_grid(M->output_type, E);
		if (!product_ok(M->output_type, E) || M->ghead <= 0 ||
		    !(is_kq(M->embd_type) ? E % 256 == 0 : E % 32 == 0)) {
			lm_err("lm_upload: E=%zu not supported by the embedding / output types %d / %d",
			       E, M->embd_type, M->output_type);
			goto fail;
		}
	}

	if (!upload_t(&M->d_wte, d->token_embd, M->embd_type, M->V, E, "upload token_embd") ||
	    !upload_t(&M->d_head, d->output, M->output_type, M->V, E, "upload output") ||
	    !upload((void **)&M->d_onorm, d->output_norm, E * sizeof(float), "upload output_norm"))
		goto fail;
	M->weight_bytes = M->V * (moe_row_bytes(M->embd_type, E) + moe_row_bytes(M->output_type, E)) +
			  E * sizeof(float);

	M->ly = calloc(M->L, sizeof(*M->ly));
	const size_t qb = qbytes(wt, M->EQ, E), kb = qbytes(wt, M->EKV, E);
	stage = malloc(qb + 2 * kb);
	if (!M->ly || !stage) {
		lm_err("lm_upload: out of host memory");
		goto fail;
	}
	for (size_t l = 0; l < M->L; l++) {
		struct lm_layer *y = &M->ly[l];
		if (!d->attn_norm[l] || !d->attn_q[l] || !d->attn_k[l] || !d->attn_v[l] ||
		    !d->attn_o[l] || !d->ffn_norm[l] || !d->gate_inp[l]) {
			lm_err("lm_upload: NULL tensor of layer %zu", l);
			goto fail;
		}
		if (!M->generic) {
			memcpy(stage, d->attn_q[l], qb);
			memcpy(stage + qb, d->attn_k[l], kb);
			memcpy(stage + qb + kb, d->attn_v[l], kb);
			if (!upload((void **)&y->wqkv, stage, qb + 2 * kb, "upload attn_q/k/v") ||
			    !upload((void **)&y->wo, d->attn_o[l], qbytes(wt, E, M->EQ),
				    "upload attn_output"))
				goto fail;
		} else {
			y->tq = layer_type(d, l, 0);
			y->tk = layer_type(d, l, 1);
			y->tv = layer_type(d, l, 2);
			y->to = layer_type(d, l, 3);
			y->gq = product_grid(y->tq, E);
			y->gk = product_grid(y->tk, E);
			y->gv = product_grid(y->tv, E);
			y->go = product_grid(y->to, M->EQ);
			if (!product_ok(y->tq, E) || !product_ok(y->tk, E) || !product_ok(y->tv, E) ||
			    !product_ok(y->to, M->EQ) || y->gq <= 0 || y->gk <= 0 || y->gv <= 0 ||
			    y->go <= 0) {
				lm_err("lm_upload: layer %zu: E=%zu / heads*128=%zu not supported by "
				       "the types %d %d %d %d", l, E, M->EQ, y->tq, y->tk, y->tv, y->to);
				goto fail;
			}
			/* q with k (and v) of its type as one matrix: every row's dot
			 * is the same whatever rows share its launch */
			y->nqkv = y->tk != y->tq ? 1 : y->tv != y->tq ? 2 : 3;
			const void *src[3] = {d->attn_q[l], d->attn_k[l], d->attn_v[l]};
			const size_t rows[3] = {M->EQ, M->EKV, M->EKV};
			if (!upload_stacked(&y->wq, src, rows, y->nqkv, y->tq, E, "upload attn_q/k/v") ||
			    (y->nqkv < 2 &&
			     !upload_t(&y->wk, d->attn_k[l], y->tk, M->EKV, E, "upload attn_k")) ||
			    (y->nqkv < 3 &&
			     !upload_t(&y->wv, d->attn_v[l], y->tv, M->EKV, E, "upload attn_v")) ||
			    !upload_t(&y->wo, d->attn_o[l], y->to, E, M->EQ, "upload attn_output"))
				goto fail;
		}
		if (!upload((void **)&y->attn_norm, d->attn_norm[l], E * 4, "upload attn_norm") ||
		    !upload((void **)&y->ffn_norm, d->ffn_norm[l], E * 4, "upload ffn_norm"))
			goto fail;
		if (d->arch == HIP_LM_OLMOE &&
		    (!upload((void **)&y->q_norm, d->q_norm[l], M->EQ * 4, "upload attn_q_norm") ||
		     !upload((void **)&y->k_norm, d->k_norm[l], M->EKV * 4, "upload attn_k_norm")))
			goto fail;
		y->moe = hip_moe_upload_typed(d->gate_inp[l], d->gate_e + l * M->NE,
					      d->up_e + l * M->NE, d->down_e + l * M->NE,
					      layer_type(d, l, 4), layer_type(d, l, 5), E, M->EI,
					      M->NE, M->K, d->arch == HIP_LM_MIXTRAL);
		if (!y->moe)
			goto fail; /* hip_moe_upload recorded why */
		/* scratch for one token now: never allocated under capture */
		if (!hip_moe_reserve(y->moe, 1))
			goto fail;
		M->weight_bytes += (M->generic ? M->EQ * moe_row_bytes(y->tq, E) +
							 M->EKV * (moe_row_bytes(y->tk, E) +
								   moe_row_bytes(y->tv, E)) +
							 E * moe_row_bytes(y->to, M->EQ)
					       : qb + 2 * kb + qbytes(wt, E, M->EQ)) +
				   2 * E * 4 + (y->q_norm ? (M->EQ + M->EKV) * 4 : 0) +
				   hip_moe_weight_bytes(y->moe);
	}
	free(stage);
	stage = NULL;

	/* rope frequencies 1 / powf(theta, 2i / HLEN) (nn.c:205), the host's libm */
	{
		float fr[LM_HLEN / 2];
		for (size_t i = 0; i < M->HL / 2; i++)
			fr[i] = 1.0f / powf(M->theta, (float)(2 * i) / (float)M->HL);
		if (!upload((void **)&M->d_freq, fr, sizeof(fr), "upload rope frequencies"))
			goto fail;
	}
	const size_t cache = M->L * M->KH * M->C * M->HL * sizeof(float);
	HIPCHK(hipMalloc((void **)&M->d_kc, cache), "hipMalloc(k cache)");
	HIPCHK(hipMalloc((void **)&M->d_vc, cache), "hipMalloc(v cache)");
	HIPCHK(hipMemset(M->d_kc, 0, cache), "clear k cache");
	HIPCHK(hipMemset(M->d_vc, 0, cache), "clear v cache");
	const size_t EA = E > M->EQ ? E : M->EQ;
	HIPCHK(hipMalloc((void **)&M->d_x, EA * 4), "hipMalloc(x)");
	HIPCHK(hipMalloc((void **)&M->d_h0, E * 4), "hipMalloc(h0)");
	HIPCHK(hipMalloc((void **)&M->d_h1, E * 4), "hipMalloc(h1)");
	HIPCHK(hipMalloc((void **)&M->d_qkv, (M->EQ + 2 * M->EKV) * 4), "hipMalloc(qkv)");
	HIPCHK(hipMalloc((void **)&M->d_attn, EA * 4), "hipMalloc(attn)");
	HIPCHK(hipMalloc((void **)&M->d_moe_in, M->L * E * 4), "hipMalloc(moe_in)");
	HIPCHK(hipMalloc((void **)&M->d_moe_out, E * 4), "hipMalloc(moe_out)");
	const size_t part = M->H * (size_t)lm_attn_chunks((int)M->C, (int)M->window) *
			    (LM_HLEN + 2) * sizeof(uint64_t);
	HIPCHK(hipMalloc((void **)&M->d_part, part), "hipMalloc(attention partials)");
	HIPCHK(hipMemset(M->d_part, 0, part), "clear attention partials");
	HIPCHK(hipMalloc((void **)&M->d_rows_t, E * sizeof(uint64_t)), "hipMalloc(rows)");
	HIPCHK(hipMemset(M->d_rows_t, 0, E * sizeof(uint64_t)), "clear rows");
	HIPCHK(hipMalloc((void **)&M->d_best, 2 * LM_MAX_HEAD_WG * sizeof(uint64_t)),
	       "hipMalloc(best)");
	HIPCHK(hipMemset(M->d_best, 0, 2 * LM_MAX_HEAD_WG * sizeof(uint64_t)), "clear best");
	HIPCHK(hipMalloc((void **)&M->d_cnt, M->H * sizeof(uint32_t)), "hipMalloc(counters)");
	HIPCHK(hipMemset(M->d_cnt, 0, M->H * sizeof(uint32_t)), "clear counters");
	HIPCHK(hipMalloc((void **)&M->d_logits, M->V * 4), "hipMalloc(logits)");
	HIPCHK(hipMalloc((void **)&M->d_ids, M->L * M->K * 4), "hipMalloc(ids)");
	HIPCHK(hipMalloc((void **)&M->d_w, M->L * M->K * 4), "hipMalloc(w)");
	HIPCHK(hipMalloc((void **)&M->d_st, sizeof(LmState)), "hipMalloc(state)");
	/* epoch 1: tags never match the zeroed gather buffers */
	M->st.epoch = 1;
	HIPCHK(hipMemcpy(M->d_st, &M->st, sizeof(LmState), hipMemcpyHostToDevice), "set state");
	{ /* the prefill rows' embedding lookups: row s takes prompt[s] */
		LmState ps;
		memset(&ps, 0, sizeof(ps));
		ps.n_prompt = 1;
		HIPCHK(hipMalloc((void **)&M->d_pst, sizeof(LmState)), "hipMalloc(prefill state)");
		HIPCHK(hipMemcpy(M->d_pst, &ps, sizeof(ps), hipMemcpyHostToDevice),
		       "set prefill state");
	}
	HIPCHK(hipDeviceSynchronize(), "synchronize after upload");
	return M;
fail:
	free(stage);
	hip_lm_free(M);
	return NULL;
}

int hip_lm_set_moe_path(hip_lm *M, int path)
{
	if (!M) {
		lm_err("lm_set_moe_path: NULL model");
		return 0;
	}
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	for (size_t l = 0; l < M->L; l++)
		if (!hip_moe_set_path(M->ly[l].moe, path))
			return 0;
	M->path_gen++; /* step graphs (the model's and its batches') hold the old launches */
	return 1;
fail:
	return 0;
}

size_t hip_lm_weight_bytes(const hip_lm *M)
{
	return M ? M->weight_bytes : 0;
}

/* the rows kvcache_rotate keeps of a full cache of `size` rows
 * (kvcache.c:36-39: the sliding window, else half the context), or 0 with
 * an error when it would keep them all: a sliding window of at least the
 * context, where the reference's next step writes its k/v row past the end
 * of its cache */
static size_t rotate_keep(const hip_lm *M, size_t size)
{
	size_t keep = M->window ? M->window : M->C / 2;
	if (keep >= size) {
		lm_err("lm: the cache is full (%zu rows) and kvcache_rotate would keep every row "
		       "(sliding window %zu, context %zu): no room for the next step", size,
		       M->window, M->C);
		return 0;
	}
	return keep;
}

/* kvcache_rotate (kvcache.c:31-56) when the cache is full, before a step;
 * the host mirror of the counters is exact (one row per step) */
static int rotate_if_full(hip_lm *M)
{
	if ((size_t)M->st.size < M->C)
		return 1;
	const size_t keep = rotate_keep(M, (size_t)M->st.size);
	if (!keep)
		return 0;
	const size_t drop = (size_t)M->st.size - keep;
	const size_t slab = M->C * M->HL, slabs = M->L * M->KH;
	if (drop > 0) {
		for (int kv = 0; kv < 2; kv++) {
			float *base = kv ? M->d_vc : M->d_kc;
			if (drop >= keep) {
				LCHK(lm_launch_copy_rows(base + drop * M->HL, base, slab, keep * M->HL,
							 slabs, M->stream), "kv rotate");
			} else { /* overlapping: row blocks of `drop` rows, front to back */
				for (size_t r = 0; r < keep; r += drop) {
					size_t n = keep - r < drop ? keep - r : drop;
					LCHK(lm_launch_copy_rows(base + (r + drop) * M->HL,
								 base + r * M->HL, slab, n * M->HL,
								 slabs, M->stream), "kv rotate");
				}
			}
		}
	}
	M->st.size = (int)keep;
	HIPCHK(hipMemcpyAsync(&M->d_st->size, &M->st.size, sizeof(int), hipMemcpyHostToDevice,
			      M->stream), "set cache size");
	/* the pageable source must stay put until the copy has been taken */
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize after rotate");
	return 1;
fail:
	return 0;
}

/* the step of a model with mixed block types (K-quants): the same stages
 * as enqueue_step's fused kernels, one launch each: the token's embedding
 * row (any type), rms_norm, the q, k and v products in their own types
 * (K-quants through Q8_K activations, bit for bit dot_q8_quant), the same
 * attention, the output product with the residual, rms_norm, the MoE layer
 * on its experts' types; then the final rms_norm, the lm_head product,
 * the greedy pick and the counters' advance */
static int enqueue_step_generic(hip_lm *M, int head, int nact)
{
	const int E = (int)M->E, EQ = (int)M->EQ, EK = (int)M->EKV;
	hipStream_t s = M->stream;
	for (size_t l = 0; l < M->L; l++) {
		struct lm_layer *y = &M->ly[l];
		const size_t co = l * M->KH * M->C * M->HL;
		/* layer 0: the token's embedding row; then h0 = h1 + moe_out */
		if (l == 0)
			LCHK(lm_launch_embed(M->embd_type, M->d_wte, E, M->d_st, M->d_prompt, M->d_h0, s),
			     "embedding");
		const float *na = l ? M->d_h1 : M->d_h0, *nb = l ? M->d_moe_out : NULL;
		float *nh = l ? M->d_h0 : NULL;
		const int nq = EQ + (y->nqkv - 1) * EK;
		/* q (with the k and v rows stacked after it) into [q | k | v], on
		 * x = rms_norm(h0): a K-quant q product normalises h0 in each of its
		 * workgroups (and writes h0 and x for the other products) */
		if (is_kq(y->tq) && moe_kq_norm_ok(y->tq, E)) {
			LCHK(moe_launch_kq_gemv_norm(y->tq, y->wq, nq, E, na, nb, y->attn_norm, nh,
						     y->nqkv < 3 ? M->d_x : NULL, M->d_qkv, y->gq, s),
			     "norm + product");
		} else {
			LCHK(lm_launch_norm_rows(1, 1, E, na, nb, y->attn_norm, nh, M->d_x, NULL, M->d_st,
						 NULL, NULL, s), "norm");
			if (!vec_product(y->tq, y->wq, nq, E, M->d_x, NULL, M->d_qkv, y->gq, s))
				return 0;
		}
		if ((y->nqkv < 2 &&
		     !vec_product(y->tk, y->wk, EK, E, M->d_x, NULL, M->d_qkv + EQ, y->gk, s)) ||
		    (y->nqkv < 3 &&
		     !vec_product(y->tv, y->wv, EK, E, M->d_x, NULL, M->d_qkv + EQ + EK, y->gv, s)))
			return 0;
		LCHK(lm_launch_attn(M->d_qkv, y->q_norm, y->k_norm, M->d_freq, M->d_st, M->d_kc + co,
				    M->d_vc + co, M->d_part, M->d_cnt, M->d_attn, (int)M->H,
				    (int)M->KH, (int)M->C, (int)M->window, M->scale,
				    M->arch != HIP_LM_OLMOE, (int)l, nact, 1, 0, s), "attention");
		/* h1 = h0 + attn . Wo^T, moe_in = rms_norm(h1): the MoE layer's
		 * decode launch normalises h1 itself where one token takes it */
		if (!vec_product(y->to, y->wo, E, EQ, M->d_attn, M->d_h0, M->d_h1, y->go, s))
			return 0;
		float *moe_in = M->d_moe_in + l * M->E;
		uint32_t *ids = M->d_ids + l * M->K;
		float *wts = M->d_w + l * M->K;
		if (moe_norm_decode_ok(y->moe)) {
			if (!moe_ffn_dev_norm(y->moe, M->d_h1, y->ffn_norm, moe_in, M->d_moe_out, ids,
					      wts, s))
				return 0;
			continue;
		}
		LCHK(lm_launch_norm_rows(1, 1, E, M->d_h1, NULL, y->ffn_norm, NULL, moe_in, NULL,
					 M->d_st, NULL, NULL, s),
		     "MoE norm");
		if (!hip_moe_ffn_dev(y->moe, moe_in, M->d_moe_out, 1, NULL, ids, wts, s))
			return 0;
	}
	if (head) { /* logits = rms_norm(h1 + moe_out) . lm_head^T, the pick */
		LCHK(lm_launch_norm_rows(1, 1, E, M->d_h1, M->d_moe_out, M->d_onorm, NULL, M->d_x, NULL,
					 M->d_st, NULL, NULL, s), "final norm");
		if (!vec_product(M->output_type, M->d_head, (int)M->V, E, M->d_x, NULL, M->d_logits,
				 M->ghead, s))
			return 0;
		LCHK(lm_launch_pick_rows(M->d_logits, 1, (int)M->V, M->d_st, &M->d_st->tok,
					 M->d_tokens, 0, s), "pick");
	}
	LCHK(lm_launch_step_end(M->d_st, s), "step end");
	return 1;
}

/* one step on M->stream; head: also the lm_head product and the pick;
 * nact: the attention chunks of this step (lm_attn_active) */
static int enqueue_step(hip_lm *M, int head, int nact)
{
	if (M->generic)
		return enqueue_step_generic(M, head, nact);
	const int wt = M->wtype, E = (int)M->E, NQKV = (int)(M->EQ + 2 * M->EKV);
	hipStream_t s = M->stream;
	uint32_t *cnt_attn = M->d_cnt;
	for (size_t l = 0; l < M->L; l++) {
		struct lm_layer *y = &M->ly[l];
		const size_t co = l * M->KH * M->C * M->HL;
		/* layer 0: the token's embedding; then h0 = h1 + moe_out (the
		 * previous layer's residual); qkv = rms_norm(h0) . Wqkv^T */
		LCHK(lm_launch_qkv(wt, y->wqkv, NQKV, E, l ? M->d_h1 : NULL, l ? M->d_moe_out : NULL,
				   y->attn_norm, M->d_h0, M->d_wte, M->d_st, M->d_prompt, M->d_qkv,
				   M->grid_qkv, s), "norm + q/k/v");
		LCHK(lm_launch_attn(M->d_qkv, y->q_norm, y->k_norm, M->d_freq, M->d_st, M->d_kc + co,
				    M->d_vc + co, M->d_part, cnt_attn, M->d_attn, (int)M->H,
				    (int)M->KH, (int)M->C, (int)M->window, M->scale,
				    M->arch != HIP_LM_OLMOE, (int)l, nact, 1, 0, s), "attention");
		/* h1 = h0 + attn . Wo^T, moe_in = rms_norm(h1): where one token
		 * takes the MoE decode kernel, its workgroups each normalise h1
		 * (no gather of h1's rows behind the output product) */
		float *moe_in = M->d_moe_in + l * M->E;
		uint32_t *ids = M->d_ids + l * M->K;
		float *wts = M->d_w + l * M->K;
		if (moe_norm_decode_ok(y->moe)) {
			LCHK(lm_launch_oproj(wt, y->wo, E, (int)M->EQ, M->d_attn, M->d_h0, M->d_h1,
					     NULL, NULL, NULL, M->d_st, (int)l, M->grid_o, s),
			     "output product");
			if (!moe_ffn_dev_norm(y->moe, M->d_h1, y->ffn_norm, moe_in, M->d_moe_out,
					      ids, wts, s))
				return 0;
			continue;
		}
		LCHK(lm_launch_oproj(wt, y->wo, E, (int)M->EQ, M->d_attn, M->d_h0, M->d_h1,
				     M->d_rows_t, y->ffn_norm, moe_in, M->d_st, (int)l, M->grid_o, s),
		     "output product + norm");
		if (!hip_moe_ffn_dev(y->moe, moe_in, M->d_moe_out, 1, NULL, ids, wts, s))
			return 0;
	}
	if (head) /* logits = rms_norm(h1 + moe_out) . lm_head^T, pick, advance */
		LCHK(lm_launch_head(wt, M->d_head, (int)M->V, E, M->d_h1, M->d_moe_out, M->d_onorm,
				    M->d_logits, M->d_best, M->d_st, M->d_tokens,
				    M->grid_head, s), "lm_head + pick");
	else
		LCHK(lm_launch_step_end(M->d_st, s), "step end");
	return 1;
}

/* the prompt and token buffers hold n ids; growing them drops the graphs
 * (their nodes name the old buffers) */
static int ensure_io(hip_lm *M, size_t n_prompt, size_t n_tokens)
{
	if (n_prompt > M->prompt_cap) {
		drop_graphs(M);
		hipFree(M->d_prompt);
		M->d_prompt = NULL;
		M->prompt_cap = 0;
		HIPCHK(hipMalloc((void **)&M->d_prompt, n_prompt * sizeof(int)), "hipMalloc(prompt)");
		M->prompt_cap = n_prompt;
	}
	if (n_tokens > M->tokens_cap) {
		drop_graphs(M);
		hipFree(M->d_tokens);
		M->d_tokens = NULL;
		M->tokens_cap = 0;
		HIPCHK(hipMalloc((void **)&M->d_tokens, n_tokens * sizeof(int)), "hipMalloc(tokens)");
		M->tokens_cap = n_tokens;
	}
	return 1;
fail:
	return 0;
}

/* set the device counters for a run of n_prompt prompt steps */
static int start_run(hip_lm *M, const int *prompt, size_t n_prompt)
{
	/* earlier steps on the (non-blocking) stream read these buffers */
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	M->st.step = 0;
	M->st.n_prompt = (int)n_prompt;
	if (n_prompt)
		HIPCHK(hipMemcpy(M->d_prompt, prompt, n_prompt * sizeof(int), hipMemcpyHostToDevice),
		       "copy prompt");
	/* the host's four counters; tok, epoch and err stay the device's */
	HIPCHK(hipMemcpy(M->d_st, &M->st, 4 * sizeof(int), hipMemcpyHostToDevice), "set state");
	return 1;
fail:
	return 0;
}

static void advance_host(hip_lm *M)
{
	M->st.step++;
	M->st.pos++;
	M->st.size++;
}

/* after the stream drains: a bounded wait of a gather or of a MoE layer's
 * decode kernel that ran out makes the run's results invalid */
static int check_errors(hip_lm *M, const char *what)
{
	int err = 0;
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	HIPCHK(hipMemcpy(&err, &M->d_st->err, sizeof(int), hipMemcpyDeviceToHost), "read error");
	if (err) {
		const int zero = 0;
		HIPCHK(hipMemcpy(&M->d_st->err, &zero, sizeof(int), hipMemcpyHostToDevice),
		       "clear error");
		lm_err("%s: a gather of the step kernels ran out of polls (%d)", what, err);
		return 0;
	}
	for (size_t l = 0; l < M->L; l++) {
		int rc = hip_moe_status(M->ly[l].moe, M->stream);
		if (rc != 0) {
			lm_err("%s: layer %zu: MoE decode wait failed (%d)", what, l, rc);
			return 0;
		}
	}
	return 1;
fail:
	return 0;
}

static int check_token(const hip_lm *M, int tok)
{
	if (tok < 0 || (size_t)tok >= M->V) {
		lm_err("lm: token %d outside the vocabulary of %zu", tok, M->V);
		return 0;
	}
	return 1;
}

/* ---------------------------------------------------------------------- */
/* prefill                                                                */
/* ---------------------------------------------------------------------- */

/* rows for a prefill of T rows in all (nseq sequences' last rows through
 * the lm_head) and the MoE layers' scratch for T tokens (synchronous, never
 * under capture; the layers count the regrowth, which the step graphs
 * check before their next replay) */
static int ensure_prefill(hip_lm *M, size_t T, size_t nseq)
{
	if (T <= M->pf_cap && nseq <= M->pf_heads)
		return 1;
	if (T < M->pf_cap)
		T = M->pf_cap;
	if (nseq < M->pf_heads)
		nseq = M->pf_heads;
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize before growing prefill rows");
	free_prefill(M);
	const size_t E = M->E, NQKV = M->EQ + 2 * M->EKV;
	HIPCHK(hipMalloc((void **)&M->d_pf_h0, T * E * 4), "hipMalloc(prefill h0)");
	HIPCHK(hipMalloc((void **)&M->d_pf_h1, T * E * 4), "hipMalloc(prefill h1)");
	HIPCHK(hipMalloc((void **)&M->d_pf_x, T * E * 4), "hipMalloc(prefill x)");
	HIPCHK(hipMalloc((void **)&M->d_pf_min, T * E * 4), "hipMalloc(prefill moe_in)");
	HIPCHK(hipMalloc((void **)&M->d_pf_mout, T * E * 4), "hipMalloc(prefill moe_out)");
	HIPCHK(hipMalloc((void **)&M->d_pf_qkv, T * NQKV * 4), "hipMalloc(prefill qkv)");
	HIPCHK(hipMalloc((void **)&M->d_pf_q, T * M->EQ * 4), "hipMalloc(prefill q)");
	HIPCHK(hipMalloc((void **)&M->d_pf_attn, T * M->EQ * 4), "hipMalloc(prefill attn)");
	{ /* the partial sums of the largest of the three products: q/k/v and
	   * output over T rows, the lm_head over the nseq last rows */
		size_t wb = moe_qmm_work_bytes((int)T, (int)NQKV, (int)E);
		const size_t w2 = moe_qmm_work_bytes((int)T, (int)E, (int)M->EQ);
		const size_t w3 = moe_qmm_work_bytes((int)nseq, (int)M->V, (int)E);
		wb = wb > w2 ? wb : w2;
		wb = wb > w3 ? wb : w3;
		if (wb)
			HIPCHK(hipMalloc(&M->d_pf_split, wb), "hipMalloc(prefill partial sums)");
	}
	for (size_t l = 0; l < M->L; l++)
		if (!hip_moe_reserve(M->ly[l].moe, T))
			return 0;
	M->pf_cap = T;
	M->pf_heads = nseq;
	return 1;
fail:
	free_prefill(M);
	return 0;
}

/* out[T][N] = add + x[T][K] . W^T (add NULL or [T][N]): the matrix cores
 * where K suits them, else the per-token product */
static int rows_product(hip_lm *M, const uint8_t *W, int N, int K, const float *x, int T,
			const float *add, float *out, hipStream_t s)
{
	const int wt = M->wtype;
	if (moe_qmm_supported(wt, K))
		LCHK(moe_launch_qmm(wt, W, N, K, x, T, add, add != NULL, out, M->d_pf_split, s),
		     "prefill product");
	else
		LCHK(moe_launch_qgemv(wt, W, N, K, x, T, add, add != NULL, out, 0, s),
		     "prefill product");
	return 1;
}

/*
 * olmoe_prefill / llama_prefill (olmoe.c:409-508, llama.c:458-564) of nseq
 * sequences at once: T ids each (sequence z's at d_ids + z * T, its cache
 * at kc / vc + z * cstride), all at cache size `size` and position `pos`,
 * as one forward of nseq * T rows: every layer on the rows (rms_norm rows,
 * the stacked q/k/v product, q/k norms and RoPE with the new k/v rows into
 * the caches, causal attention over each sequence's cache, the output
 * product with the residual, rms_norm, the MoE layer at nseq * T tokens),
 * then each sequence's last row: the final rms_norm, the lm_head product
 * into logits [nseq][V] and the greedy pick into btok[z] and, when tokens
 * is not NULL, tokens[z * tstride].  Enqueued on `s`; the caller advances
 * the position and cache size by T.
 */
static int enqueue_prefill(hip_lm *M, int size, int pos, size_t T, size_t nseq,
			   const int *d_ids, float *kc, float *vc, size_t cstride, float *logits,
			   int *btok, int *tokens, int tstride, hipStream_t s)
{
	const int wt = M->wtype, E = (int)M->E, NQKV = (int)(M->EQ + 2 * M->EKV);
	const int n = (int)(T * nseq);
	int ok = 0;
	for (size_t l = 0; l < M->L; l++) {
		struct lm_layer *y = &M->ly[l];
		const size_t co = l * M->KH * M->C * M->HL;
		/* layer 0: the ids' embedding rows; then h0 = h1 + moe_out */
		if (lm_launch_norm_rows(wt, n, E, l ? M->d_pf_h1 : NULL, l ? M->d_pf_mout : NULL,
					y->attn_norm, M->d_pf_h0, M->d_pf_x, M->d_wte, M->d_pst, d_ids,
					d_ids, s) != 0) {
			lm_err("prefill norm: launch failed");
			goto out;
		}
		if (!rows_product(M, y->wqkv, NQKV, E, M->d_pf_x, n, NULL, M->d_pf_qkv, s))
			goto out;
		if (lm_launch_pf_qk(M->d_pf_qkv, y->q_norm, y->k_norm, M->d_freq, kc + co, vc + co,
				    M->d_pf_q, (int)M->H, (int)M->KH, (int)M->C, size, pos, (int)T,
				    (int)nseq, cstride, s) != 0 ||
		    lm_launch_pf_attn(M->d_pf_q, kc + co, vc + co, M->d_pf_attn, (int)M->H,
				      (int)M->KH, (int)M->C, size, (int)T, (int)M->window, M->scale,
				      M->arch != HIP_LM_OLMOE, (int)nseq, cstride, s) != 0) {
			lm_err("prefill attention: launch failed");
			goto out;
		}
		/* h1 = h0 + attn . Wo^T, moe_in = rms_norm(h1) */
		if (!rows_product(M, y->wo, E, (int)M->EQ, M->d_pf_attn, n, M->d_pf_h0, M->d_pf_h1,
				  s))
			goto out;
		if (lm_launch_norm_rows(wt, n, E, M->d_pf_h1, NULL, y->ffn_norm, NULL, M->d_pf_min,
					NULL, M->d_pst, NULL, NULL, s) != 0) {
			lm_err("prefill MoE norm: launch failed");
			goto out;
		}
		if (!hip_moe_ffn_dev(y->moe, M->d_pf_min, M->d_pf_mout, (size_t)n, NULL, NULL, NULL, s))
			goto out;
	}
	{ /* each sequence's last row (gathered where there are several):
	   * rms_norm(h1 + moe_out) . lm_head^T and the pick */
		const size_t last = (T - 1) * M->E;
		const float *h1 = M->d_pf_h1 + last, *mo = M->d_pf_mout + last;
		if (nseq > 1) { /* into the first nseq of two spent [rows][E] buffers */
			const size_t pitch = T * M->E * 4;
			HIPCHK(hipMemcpy2DAsync(M->d_pf_h0, M->E * 4, h1, pitch, M->E * 4, nseq,
						hipMemcpyDeviceToDevice, s), "gather last rows");
			HIPCHK(hipMemcpy2DAsync(M->d_pf_min, M->E * 4, mo, pitch, M->E * 4, nseq,
						hipMemcpyDeviceToDevice, s), "gather last rows");
			h1 = M->d_pf_h0;
			mo = M->d_pf_min;
		}
		if (lm_launch_norm_rows(wt, (int)nseq, E, h1, mo, M->d_onorm, NULL, M->d_pf_x, NULL,
					M->d_pst, NULL, NULL, s) != 0) {
			lm_err("prefill final norm: launch failed");
			goto out;
		}
		if (!rows_product(M, M->d_head, (int)M->V, E, M->d_pf_x, (int)nseq, NULL, logits, s))
			goto out;
		if (lm_launch_pick_rows(logits, (int)nseq, (int)M->V, M->d_pst, btok, tokens,
					tstride, s) != 0) {
			lm_err("prefill pick: launch failed");
			goto out;
		}
	}
	ok = 1;
fail:
out:
	return ok;
}

/* a prefill of n ids fits the cache from the model's current size (the
 * reference's prefill does not rotate: past the context it writes beyond
 * its cache) */
static int prefill_fits(const hip_lm *M, size_t n)
{
	return (size_t)M->st.size + n <= M->C;
}

int hip_lm_prefill(hip_lm *M, const int *prompt, size_t n, float *logits, int *next)
{
	if (!M || !prompt || n == 0) {
		lm_err("lm_prefill: NULL argument or empty prompt");
		return 0;
	}
	for (size_t i = 0; i < n; i++)
		if (!check_token(M, prompt[i]))
			return 0;
	if (!prefill_fits(M, n)) {
		lm_err("lm_prefill: %zu ids from cache row %d do not fit the context of %zu", n,
		       M->st.size, M->C);
		return 0;
	}
	if (M->generic) {
		lm_err("lm_prefill: a model of mixed block types (K-quants) decodes its prompt "
		       "a step per id (hip_lm_decode / hip_lm_generate)");
		return 0;
	}
	if (!ensure_io(M, n, 1) || !ensure_prefill(M, n, 1))
		return 0;
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	HIPCHK(hipMemcpy(M->d_prompt, prompt, n * sizeof(int), hipMemcpyHostToDevice),
	       "copy prompt");
	if (!enqueue_prefill(M, M->st.size, M->st.pos, n, 1, M->d_prompt, M->d_kc, M->d_vc, 0,
			     M->d_logits, &M->d_st->tok, NULL, 0, M->stream))
		return 0;
	M->st.pos += (int)n;
	M->st.size += (int)n;
	if (!check_errors(M, "lm_prefill"))
		return 0;
	/* step and prompt counters belong to a run; the device's token stays */
	HIPCHK(hipMemcpy(M->d_st, &M->st, 4 * sizeof(int), hipMemcpyHostToDevice), "set state");
	if (logits)
		HIPCHK(hipMemcpy(logits, M->d_logits, M->V * 4, hipMemcpyDeviceToHost), "copy logits");
	if (next)
		HIPCHK(hipMemcpy(next, &M->d_st->tok, sizeof(int), hipMemcpyDeviceToHost),
		       "read pick");
	return 1;
fail:
	return 0;
}

int hip_lm_decode(hip_lm *M, int tok, float *logits, int *next)
{
	if (!M) {
		lm_err("lm_decode: NULL model");
		return 0;
	}
	if (!check_token(M, tok) || !ensure_io(M, 1, 1) || !rotate_if_full(M) ||
	    !start_run(M, &tok, 1) ||
	    !enqueue_step(M, 1, lm_attn_active(M->st.size, (int)M->window)))
		return 0;
	advance_host(M);
	if (!check_errors(M, "lm_decode"))
		return 0;
	if (logits)
		HIPCHK(hipMemcpy(logits, M->d_logits, M->V * 4, hipMemcpyDeviceToHost), "copy logits");
	if (next) {
		LmState st;
		HIPCHK(hipMemcpy(&st, M->d_st, sizeof(st), hipMemcpyDeviceToHost), "read state");
		*next = st.tok;
	}
	return 1;
fail:
	return 0;
}

static int capture(hip_lm *M, int head, int nact, hipGraphExec_t *out)
{
	hipGraph_t g = NULL;
	HIPCHK(hipStreamBeginCapture(M->stream, hipStreamCaptureModeThreadLocal), "begin capture");
	if (!enqueue_step(M, head, nact)) {
		hipStreamEndCapture(M->stream, &g);
		if (g)
			hipGraphDestroy(g);
		return 0;
	}
	HIPCHK(hipStreamEndCapture(M->stream, &g), "end capture");
	HIPCHK(hipGraphInstantiate(out, g, NULL, NULL, 0), "instantiate step graph");
	hipGraphDestroy(g);
	return 1;
fail:
	if (g)
		hipGraphDestroy(g);
	return 0;
}

int hip_lm_generate(hip_lm *M, const int *prompt, size_t n_prompt, size_t n_gen, int *tokens,
		    float *decode_ms)
{
	if (!M || !prompt || !tokens || n_prompt == 0) {
		lm_err("lm_generate: NULL argument or empty prompt");
		return 0;
	}
	for (size_t i = 0; i < n_prompt; i++)
		if (!check_token(M, prompt[i]))
			return 0;
	const size_t steps = n_prompt + n_gen;
	if (steps > 0x7fffffff) {
		lm_err("lm_generate: too many steps");
		return 0;
	}
	/* the prompt as one forward (olmoe_generate's olmoe_prefill,
	 * olmoe.c:556-558) where it fits the cache; else a step per id */
	const int pf = n_prompt >= 2 && prefill_fits(M, n_prompt) && !M->generic;
	if (!ensure_io(M, n_prompt, steps) || (pf && !ensure_prefill(M, n_prompt, 1)) ||
	    !start_run(M, prompt, n_prompt))
		return 0;
	size_t first = 0; /* the first step that runs a step graph */
	if (pf) {
		if (!enqueue_prefill(M, M->st.size, M->st.pos, n_prompt, 1, M->d_prompt, M->d_kc,
				     M->d_vc, 0, M->d_logits, &M->d_st->tok,
				     M->d_tokens + (n_prompt - 1), 0, M->stream))
			return 0;
		M->st.step = (int)n_prompt;
		M->st.pos += (int)n_prompt;
		M->st.size += (int)n_prompt;
		/* the prefill kernels do not read these four (the pick writes the
		 * token after them); the step graphs below do */
		HIPCHK(hipMemcpy(M->d_st, &M->st, 4 * sizeof(int), hipMemcpyHostToDevice),
		       "set state after prefill");
		first = n_prompt;
	}
	if (M->graph_gen != moe_gen(M)) {
		drop_graphs(M);
		M->graph_gen = moe_gen(M);
	}
	/* capture every step shape the run needs before its first launch: the
	 * cache size of each step is known here (one row per step, and
	 * kvcache_rotate's keep when full) */
	{
		size_t size = (size_t)M->st.size;
		for (size_t i = first; i < steps; i++) {
			if (size >= M->C && !(size = rotate_keep(M, size)))
				return 0;
			const int head = i + 1 >= n_prompt;
			const int nact = lm_attn_active((int)size, (int)M->window);
			hipGraphExec_t *ge = head ? &M->g_head[nact] : &M->g_body[nact];
			if (!*ge && !capture(M, head, nact, ge))
				return 0;
			size++;
		}
	}
	for (size_t i = first; i < steps; i++) {
		if (!rotate_if_full(M))
			return 0;
		/* prompt steps before the last need no lm_head */
		const int head = i + 1 >= n_prompt;
		const int nact = lm_attn_active(M->st.size, (int)M->window);
		hipGraphExec_t *ge = head ? &M->g_head[nact] : &M->g_body[nact];
		if (i == n_prompt)
			HIPCHK(hipEventRecord(M->ev0, M->stream), "event");
		HIPCHK(hipGraphLaunch(*ge, M->stream), "step graph");
		advance_host(M);
	}
	HIPCHK(hipEventRecord(M->ev1, M->stream), "event");
	if (!check_errors(M, "lm_generate"))
		return 0;
	if (decode_ms) {
		*decode_ms = 0.0f;
		if (n_gen)
			HIPCHK(hipEventElapsedTime(decode_ms, M->ev0, M->ev1), "event time");
	}
	HIPCHK(hipMemcpy(tokens, M->d_tokens + (n_prompt - 1), (n_gen + 1) * sizeof(int),
			 hipMemcpyDeviceToHost), "copy tokens");
	return 1;
fail:
	return 0;
}

int hip_lm_trace(hip_lm *M, float *moe_in, uint32_t *ids, float *w)
{
	if (!M) {
		lm_err("lm_trace: NULL model");
		return 0;
	}
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	if (moe_in)
		HIPCHK(hipMemcpy(moe_in, M->d_moe_in, M->L * M->E * 4, hipMemcpyDeviceToHost),
		       "copy moe_in");
	if (ids)
		HIPCHK(hipMemcpy(ids, M->d_ids, M->L * M->K * 4, hipMemcpyDeviceToHost), "copy ids");
	if (w)
		HIPCHK(hipMemcpy(w, M->d_w, M->L * M->K * 4, hipMemcpyDeviceToHost), "copy w");
	return 1;
fail:
	return 0;
}

int hip_lm_reset(hip_lm *M)
{
	if (!M) {
		lm_err("lm_reset: NULL model");
		return 0;
	}
	const size_t cache = M->L * M->KH * M->C * M->HL * sizeof(float);
	HIPCHK(hipStreamSynchronize(M->stream), "synchronize");
	HIPCHK(hipMemset(M->d_kc, 0, cache), "clear k cache");
	HIPCHK(hipMemset(M->d_vc, 0, cache), "clear v cache");
	memset(&M->st, 0, sizeof(M->st));
	/* the host's counters and tok; the epoch keeps counting */
	HIPCHK(hipMemcpy(M->d_st, &M->st, 5 * sizeof(int), hipMemcpyHostToDevice), "clear state");
	HIPCHK(hipDeviceSynchronize(), "synchronize");
	return 1;
fail:
	return 0;
}

/* ---------------------------------------------------------------------- */
/* several sequences in lockstep                                          */
/* ---------------------------------------------------------------------- */

/*
 * A step of S sequences: per layer
 *   norm rows (residual + rms_norm, or the embedding rows at layer 0) ->
 *   q/k/v product for S tokens -> attention (grid heads x chunks x S, each
 *   sequence its own cache) -> output product with the residual rows as
 *   its add operand -> rms_norm rows -> the MoE layer at T = S,
 * then the final norm rows, the lm_head product for S tokens and a
 * first-maximum pick per sequence.  Every sequence is at the same position,
 * so the step counters (LmState) are shared; the tokens are per sequence.
 */
struct hip_lm_batch {
	hip_lm *M;
	size_t S;
	hipStream_t stream;
	float *d_kc, *d_vc; /* [S][L][KH][C][HL] */
	float *d_h0, *d_h1, *d_xn, *d_moe_in, *d_moe_out; /* [S][E] */
	float *d_qkv;       /* [S][EQ + 2 EKV] */
	float *d_attn;      /* [S][EQ] */
	float *d_logits;    /* [S][V] */
	uint64_t *d_part;   /* [S][H][chunks][HL + 2] */
	uint32_t *d_cnt;    /* [S][H] */
	int *d_btok;        /* [S] each sequence's last pick */
	void *d_split;      /* the partial sums of a matrix-core product */
	LmState *d_st;
	int *d_prompt;      /* [S][n_prompt] */
	int *d_tokens;      /* [S][tokens_cap] */
	size_t prompt_cap, tokens_cap;
	LmState st;
	hipGraphExec_t *g_body, *g_head;
	unsigned graph_gen; /* the MoE layers' scratch generation the graphs name */
	hipEvent_t ev0, ev1;
};

static size_t batch_cache_floats(const hip_lm *M)
{
	return M->L * M->KH * M->C * M->HL;
}

static void batch_drop_graphs(hip_lm_batch *B)
{
	for (int i = 0; B->g_body && i <= B->M->nch; i++) {
		if (B->g_body[i])
			hipGraphExecDestroy(B->g_body[i]);
		if (B->g_head[i])
			hipGraphExecDestroy(B->g_head[i]);
		B->g_body[i] = B->g_head[i] = NULL;
	}
}

void hip_lm_batch_free(hip_lm_batch *B)
{
	if (!B)
		return;
	batch_drop_graphs(B);
	free(B->g_body);
	free(B->g_head);
	void *bufs[] = {B->d_kc, B->d_vc, B->d_h0, B->d_h1, B->d_xn, B->d_moe_in, B->d_moe_out,
			B->d_qkv, B->d_attn, B->d_logits, B->d_part, B->d_cnt, B->d_btok, B->d_st,
			B->d_prompt, B->d_tokens, B->d_split};
	for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
		hipFree(bufs[i]);
	if (B->ev0)
		hipEventDestroy(B->ev0);
	if (B->ev1)
		hipEventDestroy(B->ev1);
	if (B->stream)
		hipStreamDestroy(B->stream);
	free(B);
}

static int batch_io(hip_lm_batch *B, size_t n_prompt, size_t n_tokens);

hip_lm_batch *hip_lm_batch_new(hip_lm *M, size_t nseq)
{
	if (!M || nseq < 1 || nseq > 4096) {
		lm_err("lm_batch_new: NULL model or %zu sequences (1 .. 4096)", nseq);
		return NULL;
	}
	if (M->generic) {
		lm_err("lm_batch_new: lockstep batches take models of one block type, Q8_0 or Q4_0");
		return NULL;
	}
	hip_lm_batch *B = calloc(1, sizeof(*B));
	if (!B) {
		lm_err("lm_batch_new: out of host memory");
		return NULL;
	}
	B->M = M;
	B->S = nseq;
	B->g_body = calloc((size_t)M->nch + 1, sizeof(hipGraphExec_t));
	B->g_head = calloc((size_t)M->nch + 1, sizeof(hipGraphExec_t));
	if (!B->g_body || !B->g_head) {
		lm_err("lm_batch_new: out of host memory");
		goto fail;
	}
	const size_t S = nseq, E = M->E, NQKV = M->EQ + 2 * M->EKV;
	const size_t cache = S * batch_cache_floats(M) * sizeof(float);
	const size_t part = S * M->H * (size_t)M->nch * (LM_HLEN + 2) * sizeof(uint64_t);
	HIPCHK(hipSetDevice(M->device), "hipSetDevice");
	HIPCHK(hipStreamCreateWithFlags(&B->stream, hipStreamNonBlocking), "hipStreamCreate");
	HIPCHK(hipEventCreate(&B->ev0), "hipEventCreate");
	HIPCHK(hipEventCreate(&B->ev1), "hipEventCreate");
	HIPCHK(hipMalloc((void **)&B->d_kc, cache), "hipMalloc(batch k caches)");
	HIPCHK(hipMalloc((void **)&B->d_vc, cache), "hipMalloc(batch v caches)");
	HIPCHK(hipMemset(B->d_kc, 0, cache), "clear k caches");
	HIPCHK(hipMemset(B->d_vc, 0, cache), "clear v caches");
	HIPCHK(hipMalloc((void **)&B->d_h0, S * E * 4), "hipMalloc(h0)");
	HIPCHK(hipMalloc((void **)&B->d_h1, S * E * 4), "hipMalloc(h1)");
	HIPCHK(hipMalloc((void **)&B->d_xn, S * E * 4), "hipMalloc(xn)");
	HIPCHK(hipMalloc((void **)&B->d_moe_in, S * E * 4), "hipMalloc(moe_in)");
	HIPCHK(hipMalloc((void **)&B->d_moe_out, S * E * 4), "hipMalloc(moe_out)");
	HIPCHK(hipMalloc((void **)&B->d_qkv, S * NQKV * 4), "hipMalloc(qkv)");
	HIPCHK(hipMalloc((void **)&B->d_attn, S * M->EQ * 4), "hipMalloc(attn)");
	HIPCHK(hipMalloc((void **)&B->d_logits, S * M->V * 4), "hipMalloc(logits)");
	HIPCHK(hipMalloc((void **)&B->d_part, part), "hipMalloc(attention partials)");
	HIPCHK(hipMemset(B->d_part, 0, part), "clear attention partials");
	HIPCHK(hipMalloc((void **)&B->d_cnt, S * M->H * sizeof(uint32_t)), "hipMalloc(counters)");
	HIPCHK(hipMemset(B->d_cnt, 0, S * M->H * sizeof(uint32_t)), "clear counters");
	{ /* the largest partial sums: the lm_head's or the q/k/v product's */
		size_t wb = moe_qmm_work_bytes((int)S, (int)M->V, (int)E);
		const size_t w2 = moe_qmm_work_bytes((int)S, (int)(M->EQ + 2 * M->EKV), (int)E);
		const size_t w3 = moe_qmm_work_bytes((int)S, (int)E, (int)M->EQ);
		wb = wb > w2 ? wb : w2;
		wb = wb > w3 ? wb : w3;
		if (wb)
			HIPCHK(hipMalloc(&B->d_split, wb), "hipMalloc(partial sums)");
	}
	HIPCHK(hipMalloc((void **)&B->d_btok, S * sizeof(int)), "hipMalloc(tokens)");
	HIPCHK(hipMemset(B->d_btok, 0, S * sizeof(int)), "clear tokens");
	HIPCHK(hipMalloc((void **)&B->d_st, sizeof(LmState)), "hipMalloc(state)");
	/* epoch 1: tags never match the zeroed partials */
	B->st.epoch = 1;
	HIPCHK(hipMemcpy(B->d_st, &B->st, sizeof(LmState), hipMemcpyHostToDevice), "set state");
	/* the MoE layers' scratch for S tokens now: never allocated under capture */
	for (size_t l = 0; l < M->L; l++)
		if (!hip_moe_reserve(M->ly[l].moe, S))
			goto fail;
	/* prompts and tokens of runs up to the context long: later runs of
	 * that length reuse the captured step graphs */
	if (!batch_io(B, M->C, M->C))
		goto fail;
	HIPCHK(hipDeviceSynchronize(), "synchronize after batch setup");
	return B;
fail:
	hip_lm_batch_free(B);
	return NULL;
}

/* kvcache_rotate of every sequence's cache (they are all at one size) */
static int batch_rotate_if_full(hip_lm_batch *B)
{
	hip_lm *M = B->M;
	if ((size_t)B->st.size < M->C)
		return 1;
	const size_t keep = rotate_keep(M, (size_t)B->st.size);
	if (!keep)
		return 0;
	const size_t drop = (size_t)B->st.size - keep;
	const size_t slab = M->C * M->HL, slabs = B->S * M->L * M->KH;
	if (drop > 0) {
		for (int kv = 0; kv < 2; kv++) {
			float *base = kv ? B->d_vc : B->d_kc;
			for (size_t r = 0; r < keep; r += drop) {
				size_t n = keep - r < drop ? keep - r : drop;
				LCHK(lm_launch_copy_rows(base + (r + drop) * M->HL, base + r * M->HL,
							 slab, n * M->HL, slabs, B->stream),
				     "kv rotate");
			}
		}
	}
	B->st.size = (int)keep;
	HIPCHK(hipMemcpyAsync(&B->d_st->size, &B->st.size, sizeof(int), hipMemcpyHostToDevice,
			      B->stream), "set cache size");
	HIPCHK(hipStreamSynchronize(B->stream), "synchronize after rotate");
	return 1;
fail:
	return 0;
}

/* out[S][N] = add + x[S][K] . W^T: on the matrix cores where K suits
 * them, else the per-token product */
static int batch_product(hip_lm_batch *B, const uint8_t *W, int N, int K, const float *x,
			 const float *add, float *out)
{
	const int wt = B->M->wtype, S = (int)B->S;
	if (moe_qmm_supported(wt, K)) {
		LCHK(moe_launch_qmm(wt, W, N, K, x, S, add, add != NULL, out, B->d_split, B->stream),
		     "product");
	} else {
		LCHK(moe_launch_qgemv(wt, W, N, K, x, S, add, add != NULL, out, 0, B->stream),
		     "product");
	}
	return 1;
}

static int batch_step(hip_lm_batch *B, int head, int nact)
{
	hip_lm *M = B->M;
	const int wt = M->wtype, E = (int)M->E, S = (int)B->S;
	const int NQKV = (int)(M->EQ + 2 * M->EKV);
	const size_t cseq = batch_cache_floats(M);
	hipStream_t s = B->stream;
	for (size_t l = 0; l < M->L; l++) {
		struct lm_layer *y = &M->ly[l];
		const size_t co = l * M->KH * M->C * M->HL;
		/* layer 0: the tokens' embedding rows; then h0 = h1 + moe_out */
		LCHK(lm_launch_norm_rows(wt, S, E, l ? B->d_h1 : NULL, l ? B->d_moe_out : NULL,
					 y->attn_norm, B->d_h0, B->d_xn, M->d_wte, B->d_st,
					 B->d_prompt, B->d_btok, s), "batch norm");
		if (!batch_product(B, y->wqkv, NQKV, E, B->d_xn, NULL, B->d_qkv))
			return 0;
		LCHK(lm_launch_attn(B->d_qkv, y->q_norm, y->k_norm, M->d_freq, B->d_st, B->d_kc + co,
				    B->d_vc + co, B->d_part, B->d_cnt, B->d_attn, (int)M->H,
				    (int)M->KH, (int)M->C, (int)M->window, M->scale,
				    M->arch != HIP_LM_OLMOE, (int)l, nact, S, cseq, s),
		     "batch attention");
		/* h1 = h0 + attn . Wo^T, moe_in = rms_norm(h1): where the matrix-core
		 * product leaves partial sums, one launch adds them (the reduce's
		 * order), adds h0 and normalises */
		const int EQ = (int)M->EQ;
		if (moe_qmm_supported(wt, EQ) && moe_qmm_stretches(EQ) > 1) {
			LCHK(moe_launch_qmm_parts(wt, y->wo, E, EQ, B->d_attn, S, B->d_split, s),
			     "output product");
			LCHK(lm_launch_norm_parts(S, E, B->d_split, moe_qmm_stretches(EQ), (size_t)S * E,
						  B->d_h0, y->ffn_norm, B->d_h1, B->d_moe_in, s),
			     "batch reduce + MoE norm");
		} else {
			if (!batch_product(B, y->wo, E, EQ, B->d_attn, B->d_h0, B->d_h1))
				return 0;
			LCHK(lm_launch_norm_rows(wt, S, E, B->d_h1, NULL, y->ffn_norm, NULL,
						 B->d_moe_in, NULL, B->d_st, NULL, NULL, s),
			     "batch MoE norm");
		}
		if (!hip_moe_ffn_dev(y->moe, B->d_moe_in, B->d_moe_out, B->S, NULL, NULL, NULL, s))
			return 0;
	}
	if (head) {
		LCHK(lm_launch_norm_rows(wt, S, E, B->d_h1, B->d_moe_out, M->d_onorm, NULL, B->d_xn,
					 NULL, B->d_st, NULL, NULL, s), "batch final norm");
		if (!batch_product(B, M->d_head, (int)M->V, E, B->d_xn, NULL, B->d_logits))
			return 0;
		LCHK(lm_launch_pick_rows(B->d_logits, S, (int)M->V, B->d_st, B->d_btok, B->d_tokens,
					 (int)B->tokens_cap, s), "batch pick");
	}
	LCHK(lm_launch_step_end(B->d_st, s), "step end");
	return 1;
}

/* prompts [S][n_prompt] and tokens [S][n_tokens]; growing drops the graphs */
static int batch_io(hip_lm_batch *B, size_t n_prompt, size_t n_tokens)
{
	if (n_prompt * B->S > B->prompt_cap) {
		batch_drop_graphs(B);
		hipFree(B->d_prompt);
		B->d_prompt = NULL;
		B->prompt_cap = 0;
		HIPCHK(hipMalloc((void **)&B->d_prompt, n_prompt * B->S * sizeof(int)),
		       "hipMalloc(prompts)");
		B->prompt_cap = n_prompt * B->S;
	}
	if (n_tokens > B->tokens_cap) {
		batch_drop_graphs(B);
		hipFree(B->d_tokens);
		B->d_tokens = NULL;
		B->tokens_cap = 0;
		HIPCHK(hipMalloc((void **)&B->d_tokens, n_tokens * B->S * sizeof(int)),
		       "hipMalloc(tokens)");
		B->tokens_cap = n_tokens;
	}
	return 1;
fail:
	return 0;
}

static int batch_start(hip_lm_batch *B, const int *prompts, size_t n_prompt)
{
	HIPCHK(hipStreamSynchronize(B->stream), "synchronize");
	B->st.step = 0;
	B->st.n_prompt = (int)n_prompt;
	HIPCHK(hipMemcpy(B->d_prompt, prompts, n_prompt * B->S * sizeof(int),
			 hipMemcpyHostToDevice), "copy prompts");
	HIPCHK(hipMemcpy(B->d_st, &B->st, 4 * sizeof(int), hipMemcpyHostToDevice), "set state");
	return 1;
fail:
	return 0;
}

static int batch_errors(hip_lm_batch *B, const char *what)
{
	int err = 0;
	HIPCHK(hipStreamSynchronize(B->stream), "synchronize");
	HIPCHK(hipMemcpy(&err, &B->d_st->err, sizeof(int), hipMemcpyDeviceToHost), "read error");
	if (err) {
		const int zero = 0;
		HIPCHK(hipMemcpy(&B->d_st->err, &zero, sizeof(int), hipMemcpyHostToDevice),
		       "clear error");
		lm_err("%s: a gather of the step kernels ran out of polls (%d)", what, err);
		return 0;
	}
	for (size_t l = 0; l < B->M->L; l++) {
		int rc = hip_moe_status(B->M->ly[l].moe, B->stream);
		if (rc != 0) {
			lm_err("%s: layer %zu: MoE decode wait failed (%d)", what, l, rc);
			return 0;
		}
	}
	return 1;
fail:
	return 0;
}

static void batch_advance(hip_lm_batch *B)
{
	B->st.step++;
	B->st.pos++;
	B->st.size++;
}

int hip_lm_batch_decode(hip_lm_batch *B, const int *toks, float *logits, int *next)
{
	if (!B || !toks) {
		lm_err("lm_batch_decode: NULL argument");
		return 0;
	}
	for (size_t i = 0; i < B->S; i++)
		if (!check_token(B->M, toks[i]))
			return 0;
	if (!batch_io(B, 1, 1) || !batch_rotate_if_full(B) || !batch_start(B, toks, 1) ||
	    !batch_step(B, 1, lm_attn_active(B->st.size, (int)B->M->window)))
		return 0;
	batch_advance(B);
	if (!batch_errors(B, "lm_batch_decode"))
		return 0;
	if (logits)
		HIPCHK(hipMemcpy(logits, B->d_logits, B->S * B->M->V * 4, hipMemcpyDeviceToHost),
		       "copy logits");
	if (next)
		HIPCHK(hipMemcpy(next, B->d_btok, B->S * sizeof(int), hipMemcpyDeviceToHost),
		       "copy picks");
	return 1;
fail:
	return 0;
}

static int batch_capture(hip_lm_batch *B, int head, int nact, hipGraphExec_t *out)
{
	hipGraph_t g = NULL;
	HIPCHK(hipStreamBeginCapture(B->stream, hipStreamCaptureModeThreadLocal), "begin capture");
	if (!batch_step(B, head, nact)) {
		hipStreamEndCapture(B->stream, &g);
		if (g)
			hipGraphDestroy(g);
		return 0;
	}
	HIPCHK(hipStreamEndCapture(B->stream, &g), "end capture");
	HIPCHK(hipGraphInstantiate(out, g, NULL, NULL, 0), "instantiate step graph");
	hipGraphDestroy(g);
	return 1;
fail:
	if (g)
		hipGraphDestroy(g);
	return 0;
}

int hip_lm_batch_generate(hip_lm_batch *B, const int *prompts, size_t n_prompt, size_t n_gen,
			  int *tokens, float *decode_ms)
{
	if (!B || !prompts || !tokens || n_prompt == 0) {
		lm_err("lm_batch_generate: NULL argument or empty prompt");
		return 0;
	}
	hip_lm *M = B->M;
	for (size_t i = 0; i < n_prompt * B->S; i++)
		if (!check_token(M, prompts[i]))
			return 0;
	const size_t steps = n_prompt + n_gen;
	if (steps > 0x7fffffff || steps * B->S > 0x7fffffff) {
		lm_err("lm_batch_generate: too many steps");
		return 0;
	}
	/* the prompts as prefills of groups of sequences (~PF_GROUP_ROWS rows:
	 * every MoE layer's scratch grows with the rows of one launch) where
	 * they fit the caches; else a step per id */
	const int pf = n_prompt >= 2 && (size_t)B->st.size + n_prompt <= M->C;
	size_t gseq = n_prompt >= PF_GROUP_ROWS ? 1 : PF_GROUP_ROWS / n_prompt;
	gseq = gseq < B->S ? gseq : B->S;
	if (!batch_io(B, n_prompt, steps) || (pf && !ensure_prefill(M, gseq * n_prompt, gseq)) ||
	    !batch_start(B, prompts, n_prompt))
		return 0;
	size_t first = 0; /* the first step that runs a step graph */
	if (pf) {
		const size_t cseq = batch_cache_floats(M);
		for (size_t z0 = 0; z0 < B->S; z0 += gseq) {
			const size_t gz = B->S - z0 < gseq ? B->S - z0 : gseq;
			if (!enqueue_prefill(M, B->st.size, B->st.pos, n_prompt, gz,
					     B->d_prompt + z0 * n_prompt, B->d_kc + z0 * cseq,
					     B->d_vc + z0 * cseq, cseq, B->d_logits + z0 * M->V,
					     B->d_btok + z0,
					     B->d_tokens + z0 * B->tokens_cap + (n_prompt - 1),
					     (int)B->tokens_cap, B->stream))
				return 0;
		}
		B->st.step = (int)n_prompt;
		B->st.pos += (int)n_prompt;
		B->st.size += (int)n_prompt;
		/* the prefills do not read the batch's state; the step graphs do */
		HIPCHK(hipMemcpy(B->d_st, &B->st, 4 * sizeof(int), hipMemcpyHostToDevice),
		       "set state after prefill");
		first = n_prompt;
	}
	if (B->graph_gen != moe_gen(M)) { /* another batch grew the layers' scratch */
		batch_drop_graphs(B);
		B->graph_gen = moe_gen(M);
	}
	/* every step shape of the run, captured before its first launch */
	{
		size_t size = (size_t)B->st.size;
		for (size_t i = first; i < steps; i++) {
			if (size >= M->C && !(size = rotate_keep(M, size)))
				return 0;
			const int head = i + 1 >= n_prompt;
			const int nact = lm_attn_active((int)size, (int)M->window);
			hipGraphExec_t *ge = head ? &B->g_head[nact] : &B->g_body[nact];
			if (!*ge && !batch_capture(B, head, nact, ge))
				return 0;
			size++;
		}
	}
	for (size_t i = first; i < steps; i++) {
		if (!batch_rotate_if_full(B))
			return 0;
		const int head = i + 1 >= n_prompt;
		const int nact = lm_attn_active(B->st.size, (int)M->window);
		hipGraphExec_t *ge = head ? &B->g_head[nact] : &B->g_body[nact];
		if (i == n_prompt)
			HIPCHK(hipEventRecord(B->ev0, B->stream), "event");
		HIPCHK(hipGraphLaunch(*ge, B->stream), "step graph");
		batch_advance(B);
	}
	HIPCHK(hipEventRecord(B->ev1, B->stream), "event");
	if (!batch_errors(B, "lm_batch_generate"))
		return 0;
	if (decode_ms) {
		*decode_ms = 0.0f;
		if (n_gen)
			HIPCHK(hipEventElapsedTime(decode_ms, B->ev0, B->ev1), "event time");
	}
	for (size_t q = 0; q < B->S; q++)
		HIPCHK(hipMemcpy(tokens + q * (n_gen + 1), B->d_tokens + q * B->tokens_cap + (n_prompt - 1),
				 (n_gen + 1) * sizeof(int), hipMemcpyDeviceToHost), "copy tokens");
	return 1;
fail:
	return 0;
}

int hip_lm_batch_reset(hip_lm_batch *B)
{
	if (!B) {
		lm_err("lm_batch_reset: NULL batch");
		return 0;
	}
	const size_t cache = B->S * batch_cache_floats(B->M) * sizeof(float);
	HIPCHK(hipStreamSynchronize(B->stream), "synchronize");
	HIPCHK(hipMemset(B->d_kc, 0, cache), "clear k caches");
	HIPCHK(hipMemset(B->d_vc, 0, cache), "clear v caches");
	memset(&B->st, 0, sizeof(B->st));
	HIPCHK(hipMemcpy(B->d_st, &B->st, 5 * sizeof(int), hipMemcpyHostToDevice), "clear state");
	HIPCHK(hipDeviceSynchronize(), "synchronize");
	return 1;
fail:
	return 0;
}
