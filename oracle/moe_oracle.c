/*
 * CPU oracle for the quantized mixture-of-experts FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, loaded by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py.
 * The product library never links or calls it.
 *
 * A plain-C restatement of hoathienvu8x/llm.c's CPU path as built for AVX2
 * (8 fp32 lanes).  It is compiled with -ffp-contract=off and spells every
 * fused multiply-add as fmaf(), so the operation order below is the order the
 * reference executes:
 *   - lane accumulators acc[l] += a[i+l]*b[i+l] via FMA   (vector_avx2.h:121)
 *   - horizontal sum ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (vector_avx2.h:126-132)
 *   - scalar tails use `sum += a*b`, which clang contracts to an FMA under
 *     its default -ffp-contract=on (matmul.c:102-103, 233-237)
 *   - expf is glibc's scalar expf                          (vector_avx2.h:50-63)
 *
 * Parity pins (tests/test_oracle.py): router logits, softmax probabilities,
 * top-k ids/weights and layer outputs are checked bit-for-bit against golden
 * vectors produced by the compiled reference (tests/golden/); dots and
 * dequantization are also checked against float64 closed forms; top_k against
 * the reference's own known-answer test (test/nn.c:5-33) and brute force.
 */
#define _GNU_SOURCE
#include "moe_oracle.h"
#include "oracle_pool.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define LANES 8  /* AVX2_BATCH, vector_avx2.h:13 */
#define QK 32    /* GGML_QK, quant.h:11 */
#define QKK 256  /* QK_K, quant.h:28 */

/* f16 -> f32 is exact (F16C _cvtsh_ss, quant.h:71-75). */
static float h2f(uint16_t h)
{
	uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
	uint32_t e = (h >> 10) & 0x1f;
	uint32_t m = h & 0x3ff;
	uint32_t f;

	if (e == 0) {
		if (m == 0) {
			f = sign;
		} else {
			int sh = 0;
			while (!(m & 0x400)) {
				m <<= 1;
				sh++;
			}
			m &= 0x3ff;
			f = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
		}
	} else if (e == 0x1f) {
		f = sign | 0x7f800000u | (m << 13);
	} else {
		f = sign | ((e + 127 - 15) << 23) | (m << 13);
	}
	float r;
	memcpy(&r, &f, 4);
	return r;
}

static uint16_t rd16(const uint8_t *p)
{
	return (uint16_t)(p[0] | (p[1] << 8));
}

/* vector_avx2.h:126-132 */
static float lane_sum(const float a[LANES])
{
	float v0 = a[0] + a[4], v1 = a[1] + a[5], v2 = a[2] + a[6], v3 = a[3] + a[7];
	float w0 = v0 + v2, w1 = v1 + v3;
	return w0 + w1;
}

/* matmul.c:91-105 dot_f32_f32 */
static float dot_f32(const float *x, const float *y, size_t n)
{
	float acc[LANES] = {0};
	size_t nv = n - n % LANES;
	for (size_t i = 0; i < nv; i += LANES)
		for (int l = 0; l < LANES; l++)
			acc[l] = fmaf(x[i + l], y[i + l], acc[l]);
	float sum = lane_sum(acc);
	for (size_t i = nv; i < n; i++)
		sum = fmaf(x[i], y[i], sum);
	return sum;
}

float orc_dot_f32(const float *x, const float *y, size_t n)
{
	return dot_f32(x, y, n);
}

struct router_job {
	const float *x, *wr, *bias;
	size_t T, E, NE;
	float *logits;
};

/* thread tidx takes a contiguous chunk of the T * NE logits */
static void router_task(void *arg, int tidx, int nt)
{
	const struct router_job *w = arg;
	const size_t n = w->T * w->NE, chunk = (n + nt - 1) / nt;
	const size_t i0 = tidx * chunk, i1 = i0 + chunk < n ? i0 + chunk : n;
	for (size_t i = i0; i < i1; i++) {
		const size_t t = i / w->NE, j = i % w->NE;
		float init = w->bias ? w->bias[j] : 0.0f;
		w->logits[i] = init + dot_f32(&w->x[t * w->E], &w->wr[j * w->E], w->E);
	}
}

void orc_router(const float *x, const float *wr, const float *bias,
		size_t T, size_t E, size_t NE, float *logits)
{
	/* mma_init (matmul.c:13-33) seeds with the bias row or zero; the GEMV
	 * (matmul.c:115-118) and the tiled path (matmul.c:213-238) then add one
	 * complete dot per element, in the same per-element order. */
	struct router_job w = {x, wr, bias, T, E, NE, logits};
	orc_pool_run(router_task, &w, orc_pool_threads(T, E, NE));
}

/* tensor.c:479-517 (value only) */
static float row_max(const float *v, size_t n)
{
	float mx = v[0];
	size_t nv = n - n % LANES;
	for (size_t i = 0; i < nv; i += LANES) {
		float r = v[i];
		for (int l = 1; l < LANES; l++)
			if (v[i + l] > r)
				r = v[i + l];
		if (r > mx)
			mx = r;
	}
	for (size_t i = nv; i < n; i++)
		if (v[i] > mx)
			mx = v[i];
	return mx;
}

void orc_softmax_1d(float *t, size_t n)
{
	float mx = row_max(t, n);
	float vsum[LANES] = {0};
	size_t nv = n - n % LANES;

	for (size_t i = 0; i < nv; i += LANES)
		for (int l = 0; l < LANES; l++) {
			float e = expf(t[i + l] - mx);
			t[i + l] = e;
			vsum[l] = vsum[l] + e;
		}
	float sum = lane_sum(vsum);
	for (size_t i = nv; i < n; i++) {
		t[i] = expf(t[i] - mx);
		sum += t[i];
	}
	for (size_t i = 0; i < n; i++)
		t[i] = t[i] / sum;
}

void orc_top_k(const float *f, size_t n, uint32_t *ids, float *w, size_t k)
{
	for (size_t i = 0; i < k; i++) {
		ids[i] = 0;
		w[i] = f[0];
	}
	for (size_t i = 1; i < n; i++) {
		float v = f[i];
		long p = -1;
		for (size_t j = 0; j < k; j++)
			if (v > w[j])
				p = (long)j;
		if (p < 0)
			continue;
		for (long j = 0; j < p; j++) {
			ids[j] = ids[j + 1];
			w[j] = w[j + 1];
		}
		ids[p] = (uint32_t)i;
		w[p] = v;
	}
}

/* quant.c:103-124: per block, lanes l take elements g+l for g = 0,8,16,24. */
static float dot_q8_0(const float *x, const uint8_t *row, size_t n)
{
	float acc[LANES] = {0};
	for (size_t b = 0; b < n / QK; b++) {
		const uint8_t *blk = row + b * 34;
		float d = h2f(rd16(blk));
		const int8_t *qs = (const int8_t *)(blk + 2);
		for (int g = 0; g < QK; g += LANES)
			for (int l = 0; l < LANES; l++) {
				float sq = d * (float)qs[g + l];
				acc[l] = fmaf(sq, x[b * QK + g + l], acc[l]);
			}
	}
	return lane_sum(acc);
}

/* quant.c:126-155: per block, g = 0,8: low nibble of qs[g+l] with x[g+l],
 * then high nibble of qs[g+l] with x[g+16+l]; both biased by -8. */
static float dot_q4_0(const float *x, const uint8_t *row, size_t n)
{
	float acc[LANES] = {0};
	for (size_t b = 0; b < n / QK; b++) {
		const uint8_t *blk = row + b * 18;
		float d = h2f(rd16(blk));
		const uint8_t *qs = blk + 2;
		for (int g = 0; g < QK / 2; g += LANES) {
			for (int l = 0; l < LANES; l++) {
				float lo = (float)((int)(qs[g + l] & 0x0f) - 8);
				float hi = (float)((int)(qs[g + l] >> 4) - 8);
				acc[l] = fmaf(d * lo, x[b * QK + g + l], acc[l]);
				acc[l] = fmaf(d * hi, x[b * QK + g + QK / 2 + l], acc[l]);
			}
		}
	}
	return lane_sum(acc);
}

static size_t row_bytes(int wtype, size_t n)
{
	switch (wtype) {
	case ORC_Q8_0: return (n / QK) * 34;
	case ORC_Q4_0: return (n / QK) * 18;
	case ORC_Q4_K: return (n / QKK) * 144;
	case ORC_Q6_K: return (n / QKK) * 210;
	}
	abort();
}

static float dot_q4_K_f32(const float *x, const uint8_t *row, size_t n);
static float dot_q6_K_f32(const float *x, const uint8_t *row, size_t n);

float orc_dot_quant(const float *x, const void *qrow, int wtype, size_t n)
{
	if (wtype == ORC_Q8_0)
		return dot_q8_0(x, qrow, n);
	if (wtype == ORC_Q4_0)
		return dot_q4_0(x, qrow, n);
	if (wtype == ORC_Q4_K)
		return dot_q4_K_f32(x, qrow, n);
	if (wtype == ORC_Q6_K)
		return dot_q6_K_f32(x, qrow, n);
	abort();
}

/*
 * tensor_mma_transposed_2x2 with a Q8_0/Q4_0 right operand, as the
 * reference's default build (-DQ8_DOT, Makefile:29) runs it when K % 256 ==
 * 0: mma_init (matmul.c:13-33) seeds out with add ([T][N] copied, or [N] for
 * every row) or zero, then each element gets += dot_q8_quant
 * (matmul.c:107-131 for T = 1, 145-165 for T > 1), which for Q8_0/Q4_0 is
 * dot_f32_quant (quant.c:656-668, 577-614).
 */
struct qmat_job {
	const float *x;
	const void *q;
	int wtype;
	size_t T, N, K;
	const float *add;
	size_t add_len;
	float *out;
	float *q8d;     /* K-quants: the tokens in Q8_K, [T][K/256] scales, */
	int8_t *q8s;    /* [T][K] quants */
	int16_t *q8b;   /* [T][K/256][16] sums of 16 */
};

/* thread tidx of nt takes output columns [tidx * ceil(N/nt), ...) of every
 * token (transposed_gemv_thread_fn, matmul.c:107-114; for K-quants the
 * Q8_K dots of matmul.c:121-124,145-165 on the tokens quantized once) */
static void qmat_task(void *arg, int tidx, int nt)
{
	const struct qmat_job *w = arg;
	const size_t rb = row_bytes(w->wtype, w->K), chunk = (w->N + nt - 1) / nt;
	const size_t j0 = tidx * chunk, j1 = j0 + chunk < w->N ? j0 + chunk : w->N;
	const size_t nb = w->K / QKK;
	for (size_t t = 0; t < w->T; t++)
		for (size_t j = j0; j < j1; j++) {
			float init = !w->add ? 0.0f
					     : w->add_len == w->N ? w->add[j] : w->add[t * w->N + j];
			const uint8_t *qr = (const uint8_t *)w->q + j * rb;
			float dot = w->q8d ? orc_dot_q8k(w->q8d + t * nb, w->q8s + t * w->K,
							 w->q8b + t * nb * 16, qr, w->wtype, w->K)
					   : orc_dot_quant(&w->x[t * w->K], qr, w->wtype, w->K);
			w->out[t * w->N + j] = init + dot;
		}
}

void orc_qmat_mul(const float *x, size_t T, const void *q, int wtype, size_t N, size_t K,
		  const float *add, size_t add_len, float *out)
{
	struct qmat_job w = {x, q, wtype, T, N, K, add, add_len, out, NULL, NULL, NULL};
	/* the default -DQ8_DOT build quantizes the tokens to Q8_K once when
	 * K % 256 == 0 (matmul.c:291-297); dot_q8_quant takes the integer dots
	 * for K-quants and the fp32 dots otherwise (quant.c:656-668) */
	const int kq = (wtype == ORC_Q4_K || wtype == ORC_Q6_K) && K % QKK == 0;
	if (kq) {
		w.q8d = malloc(T * (K / QKK) * sizeof(float));
		w.q8s = malloc(T * K);
		w.q8b = malloc(T * (K / QKK) * 16 * sizeof(int16_t));
		for (size_t t = 0; t < T; t++)
			orc_quantize_q8k(x + t * K, K, w.q8d + t * (K / QKK), w.q8s + t * K,
					 w.q8b + t * (K / QKK) * 16);
	}
	orc_pool_run(qmat_task, &w, orc_pool_threads(T, K, N));
	if (kq) {
		free(w.q8d);
		free(w.q8s);
		free(w.q8b);
	}
}

static void dequant_kquant(const uint8_t *row, int wtype, float *dst, size_t n);

void orc_dequant_row(const void *qrow, int wtype, float *dst, size_t n)
{
	const uint8_t *row = qrow;
	for (size_t b = 0; b < n / QK; b++) {
		if (wtype == ORC_Q8_0) {
			const uint8_t *blk = row + b * 34;
			float d = h2f(rd16(blk));
			for (int j = 0; j < QK; j++)
				dst[b * QK + j] = d * (float)(int8_t)blk[2 + j];
		} else if (wtype == ORC_Q4_0) {
			const uint8_t *blk = row + b * 18;
			float d = h2f(rd16(blk));
			for (int j = 0; j < QK / 2; j++) {
				dst[b * QK + j] = d * (float)((int)(blk[2 + j] & 0x0f) - 8);
				dst[b * QK + j + QK / 2] = d * (float)((int)(blk[2 + j] >> 4) - 8);
			}
		} else if (wtype == ORC_Q4_K || wtype == ORC_Q6_K) {
			dequant_kquant(row, wtype, dst, n);
			return;
		} else {
			abort();
		}
	}
}

struct ffn_job {
	const float *x;
	const uint8_t *g8, *u8, *d8;
	int gt, dt; /* gate/up and down block types */
	size_t E, EI;
	float *h, *out;
	const float *q8d; /* K-quant gate/up: x in Q8_K */
	const int8_t *q8s;
	const int16_t *q8b;
};

static int is_kq(int t)
{
	return t == ORC_Q4_K || t == ORC_Q6_K;
}

/* nn.c:455-478: thread tidx's chunk of gate/up rows, then SwiGLU in place;
 * dot_q8_quant takes the integer dots for K-quant rows, the fp32 ones
 * otherwise (quant.c:656-668) */
static void ffn_gateup_task(void *arg, int tidx, int nt)
{
	const struct ffn_job *w = arg;
	const size_t rb_in = row_bytes(w->gt, w->E), chunk = (w->EI + nt - 1) / nt;
	const size_t j0 = tidx * chunk, j1 = j0 + chunk < w->EI ? j0 + chunk : w->EI;
	for (size_t j = j0; j < j1; j++) {
		float g, u;
		if (w->q8d) {
			g = orc_dot_q8k(w->q8d, w->q8s, w->q8b, w->g8 + j * rb_in, w->gt, w->E);
			u = orc_dot_q8k(w->q8d, w->q8s, w->q8b, w->u8 + j * rb_in, w->gt, w->E);
		} else {
			g = orc_dot_quant(w->x, w->g8 + j * rb_in, w->gt, w->E);
			u = orc_dot_quant(w->x, w->u8 + j * rb_in, w->gt, w->E);
		}
		w->h[j] = (g / (1.0f + expf(-g))) * u;
	}
}

/* nn.c:483-492: after the barrier, thread tidx's chunk of down rows (fp32
 * dots: h is not quantized) */
static void ffn_down_task(void *arg, int tidx, int nt)
{
	const struct ffn_job *w = arg;
	const size_t rb_mid = row_bytes(w->dt, w->EI), chunk = (w->E + nt - 1) / nt;
	const size_t i0 = tidx * chunk, i1 = i0 + chunk < w->E ? i0 + chunk : w->E;
	for (size_t i = i0; i < i1; i++)
		w->out[i] = orc_dot_quant(w->h, w->d8 + i * rb_mid, w->dt, w->EI);
}

void orc_fused_ffn(const float *x, const void *gate, const void *up,
		   const void *down, int wtype, size_t E, size_t EI,
		   float *h, float *out)
{
	const int gt = wtype & 0xff, dt = (wtype >> 8) ? (wtype >> 8) : gt;
	struct ffn_job w = {x, gate, up, down, gt, dt, E, EI, h, out, NULL, NULL, NULL};
	/* the -DQ8_DOT build quantizes the token to Q8_K when E % 256 == 0
	 * (nn.c:527-531) */
	float *q8d = NULL;
	int8_t *q8s = NULL;
	int16_t *q8b = NULL;
	if (is_kq(gt) && E % QKK == 0) {
		q8d = malloc(E / QKK * sizeof(float));
		q8s = malloc(E);
		q8b = malloc(E / QKK * 16 * sizeof(int16_t));
		orc_quantize_q8k(x, E, q8d, q8s, q8b);
		w.q8d = q8d;
		w.q8s = q8s;
		w.q8b = q8b;
	}
	/* fused_ffn_silu's thread_pool_run(.., 1, k, inter) (nn.c:534) */
	const int nt = orc_pool_threads(1, E, EI);
	orc_pool_run(ffn_gateup_task, &w, nt);
	orc_pool_run(ffn_down_task, &w, nt);
	free(q8d);
	free(q8s);
	free(q8b);
}

struct moe_job {
	const float *x;
	float *out;
	const float *logits;
	const void *const *gate_e, *const *up_e, *const *down_e;
	int wtype;
	size_t E, EI, NE, topk;
	int renorm;
	uint32_t *ids_out;
	float *w_out, *probs_out;
	size_t t0, t1;
};

static void moe_tokens(struct moe_job *j)
{
	size_t E = j->E, EI = j->EI, NE = j->NE, K = j->topk;
	float *probs = malloc(NE * sizeof(float));
	float *h = malloc(EI * sizeof(float));
	float *y = malloc(E * sizeof(float));
	uint32_t *ids = malloc(K * sizeof(uint32_t));
	float *w = malloc(K * sizeof(float));

	for (size_t t = j->t0; t < j->t1; t++) {
		memcpy(probs, &j->logits[t * NE], NE * sizeof(float));
		orc_softmax_1d(probs, NE);
		if (j->probs_out)
			memcpy(&j->probs_out[t * NE], probs, NE * sizeof(float));
		orc_top_k(probs, NE, ids, w, K);

		if (j->renorm) { /* llama.c:422-427 */
			float s = 0.0f;
			for (size_t e = 0; e < K; e++)
				s += w[e];
			for (size_t e = 0; e < K; e++)
				w[e] /= s;
		}
		if (j->ids_out)
			memcpy(&j->ids_out[t * K], ids, K * sizeof(uint32_t));
		if (j->w_out)
			memcpy(&j->w_out[t * K], w, K * sizeof(float));

		float *o = &j->out[t * E];
		memset(o, 0, E * sizeof(float)); /* tensor_set(output, 0), olmoe.c:357 */
		for (size_t e = 0; e < K; e++) {
			uint32_t id = ids[e];
			orc_fused_ffn(&j->x[t * E], j->gate_e[id], j->up_e[id],
				      j->down_e[id], j->wtype, E, EI, h, y);
			/* tensor_div_scalar(.., 1/w) then tensor_add, olmoe.c:401-403 */
			float inv = 1.0f / w[e];
			for (size_t i = 0; i < E; i++)
				o[i] = o[i] + y[i] / inv;
		}
	}
	free(probs);
	free(h);
	free(y);
	free(ids);
	free(w);
}

static void *moe_thread(void *arg)
{
	moe_tokens(arg);
	return NULL;
}

void orc_moe_ffn(const float *x, float *out, size_t T,
		 const float *wr, const float *bias,
		 const void *const *gate_e, const void *const *up_e,
		 const void *const *down_e, int wtype,
		 size_t E, size_t EI, size_t NE, size_t topk, int renorm,
		 uint32_t *ids_out, float *w_out, float *logits_out,
		 float *probs_out, int nthreads)
{
	float *logits = logits_out ? logits_out : malloc(T * NE * sizeof(float));
	orc_router(x, wr, bias, T, E, NE, logits);

	if (nthreads < 1 || orc_pool_active())
		nthreads = 1; /* the pool threads each operation instead */
	if ((size_t)nthreads > T)
		nthreads = (int)T;
	struct moe_job *jobs = calloc((size_t)nthreads, sizeof(*jobs));
	pthread_t *th = calloc((size_t)nthreads, sizeof(*th));
	size_t chunk = (T + nthreads - 1) / nthreads;

	for (int i = 0; i < nthreads; i++) {
		struct moe_job *j = &jobs[i];
		j->x = x;
		j->out = out;
		j->logits = logits;
		j->gate_e = gate_e;
		j->up_e = up_e;
		j->down_e = down_e;
		j->wtype = wtype;
		j->E = E;
		j->EI = EI;
		j->NE = NE;
		j->topk = topk;
		j->renorm = renorm;
		j->ids_out = ids_out;
		j->w_out = w_out;
		j->probs_out = probs_out;
		j->t0 = i * chunk < T ? i * chunk : T;
		j->t1 = (i + 1) * chunk < T ? (i + 1) * chunk : T;
	}
	if (nthreads == 1) {
		moe_tokens(&jobs[0]);
	} else {
		for (int i = 0; i < nthreads; i++)
			pthread_create(&th[i], NULL, moe_thread, &jobs[i]);
		for (int i = 0; i < nthreads; i++)
			pthread_join(th[i], NULL);
	}
	free(jobs);
	free(th);
	if (!logits_out)
		free(logits);
}

void orc_expf_array(const float *in, float *out, size_t n)
{
	for (size_t i = 0; i < n; i++)
		out[i] = expf(in[i]);
}

struct expf_job {
	uint32_t b0;
	size_t n;
	float *out;
};

static void *expf_thread(void *arg)
{
	struct expf_job *j = arg;
	for (size_t i = 0; i < j->n; i++) {
		uint32_t b = j->b0 + (uint32_t)i;
		float x;
		memcpy(&x, &b, 4);
		j->out[i] = expf(x);
	}
	return NULL;
}

void orc_expf_bits(uint32_t bits0, size_t n, float *out, int nthreads)
{
	if (nthreads < 1)
		nthreads = 1;
	struct expf_job *jobs = calloc((size_t)nthreads, sizeof(*jobs));
	pthread_t *th = calloc((size_t)nthreads, sizeof(*th));
	size_t chunk = (n + nthreads - 1) / nthreads;
	for (int i = 0; i < nthreads; i++) {
		size_t s = (size_t)i * chunk < n ? (size_t)i * chunk : n;
		size_t e = s + chunk < n ? s + chunk : n;
		jobs[i].b0 = bits0 + (uint32_t)s;
		jobs[i].n = e - s;
		jobs[i].out = out + s;
		pthread_create(&th[i], NULL, expf_thread, &jobs[i]);
	}
	for (int i = 0; i < nthreads; i++)
		pthread_join(th[i], NULL);
	free(jobs);
	free(th);
}

/* ---------------------------------------------------------------------- */
/* K-quants: Q4_K (144-byte blocks of 256), Q6_K (210-byte blocks of 256)  */
/* and the Q8_K activation blocks of the -DQ8_DOT build                    */
/* ---------------------------------------------------------------------- */

/* get_scale_min_k4 (quant.h:63-73): sub-block j's 6-bit scale and min */
static void scale_min_k4(int j, const uint8_t *q, int *d, int *m)
{
	if (j < 4) {
		*d = q[j] & 63;
		*m = q[j + 4] & 63;
	} else {
		*d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
		*m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
	}
}

/*
 * quantize_row_q8 (quant.c:627-654): per 256 values, mval = the first value
 * of largest magnitude, iscale = -127 / mval, d = 1 / iscale, q =
 * min(127, (int)roundf(iscale * x)), bsums = sums of 16 quants; an all-zero
 * block is all zero.
 */
void orc_quantize_q8k(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums)
{
	for (size_t i = 0; i < n / QKK; i++) {
		const float *xb = x + i * QKK;
		float amax = 0, mval = 0;
		for (int j = 0; j < QKK; j++) {
			float a = fabsf(xb[j]);
			if (a > amax) {
				amax = a;
				mval = xb[j];
			}
		}
		if (amax == 0) {
			d[i] = 0.0f;
			memset(qs + i * QKK, 0, QKK);
			memset(bsums + i * 16, 0, 16 * sizeof(int16_t));
			continue;
		}
		float iscale = -127.0f / mval;
		d[i] = 1.0f / iscale;
		for (int j = 0; j < QKK; j++) {
			int v = (int)roundf(iscale * xb[j]);
			qs[i * QKK + j] = (int8_t)(v < 127 ? v : 127);
		}
		for (int j = 0; j < 16; j++) {
			int sum = 0;
			for (int k = 0; k < 16; k++)
				sum += qs[i * QKK + j * 16 + k];
			bsums[i * 16 + j] = (int16_t)sum;
		}
	}
}

/*
 * dot_q4_K_q8_K (quant_cpu.h:7-60, which quant_avx2.h:8-106 equals bit for
 * bit): per super-block the exact integer sums sumi = sum over sub-blocks of
 * scale * sum(q4 * q8) and min_sum = sum over sub-blocks of min * (bsum pair),
 * then acc = fma(yd * d, sumi, acc) and acc_m = fma(-yd * dmin, min_sum,
 * acc_m) (clang -ffp-contract=on fuses `acc += d * sumi`); the result is
 * acc + acc_m.  dot_q6_K_q8_K (quant_cpu.h:62-120): sumi =
 * sum over 16-value groups of scale * sum((q6 - 32) * q8); acc += (yd * d) *
 * sumi.
 */
float orc_dot_q8k(const float *yd, const int8_t *q8, const int16_t *bsums, const void *qrow,
		  int wtype, size_t n)
{
	const uint8_t *row = qrow;
	float acc = 0, acc_m = 0;
	for (size_t i = 0; i < n / QKK; i++) {
		const int8_t *y = q8 + i * QKK;
		if (wtype == ORC_Q4_K) {
			const uint8_t *b = row + i * 144;
			const float d = yd[i] * h2f(rd16(b)), dmin = -yd[i] * h2f(rd16(b + 2));
			const uint8_t *sc = b + 4, *qs = b + 16;
			int32_t sumi = 0, min_sum = 0;
			for (int j = 0; j < 4; j++) {
				int s1, m1, s2, m2;
				scale_min_k4(2 * j, sc, &s1, &m1);
				scale_min_k4(2 * j + 1, sc, &s2, &m2);
				int32_t a = 0, c = 0;
				for (int k = 0; k < 32; k++) {
					a += (qs[j * 32 + k] & 0xF) * y[j * 64 + k];
					c += (qs[j * 32 + k] >> 4) * y[j * 64 + 32 + k];
				}
				sumi += s1 * a + s2 * c;
				min_sum += m1 * (bsums[i * 16 + 4 * j] + bsums[i * 16 + 4 * j + 1]) +
					   m2 * (bsums[i * 16 + 4 * j + 2] + bsums[i * 16 + 4 * j + 3]);
			}
			/* the reference's clang build contracts both updates into FMAs */
			acc_m = fmaf(dmin, (float)min_sum, acc_m);
			acc = fmaf(d, (float)sumi, acc);
		} else {
			const uint8_t *b = row + i * 210;
			const uint8_t *ql = b, *qh = b + 128;
			const int8_t *sc = (const int8_t *)(b + 192);
			const float d = yd[i] * h2f(rd16(b + 208));
			int32_t sumi = 0;
			for (int c = 0; c < 2; c++)
				for (int g = 0; g < 4; g++) /* 32 values: ql low/high nibble, qh 2 bits */
					for (int half = 0; half < 2; half++) {
						int32_t s = 0;
						for (int k = 0; k < 16; k++) {
							const int l = half * 16 + k;
							const int lo = g & 1 ? ql[c * 64 + 32 + l]
									     : ql[c * 64 + l];
							const int q = ((g < 2 ? lo & 0xF : lo >> 4) |
								       (((qh[c * 32 + l] >> (2 * g)) & 3) << 4)) -
								      32;
							s += q * y[c * 128 + g * 32 + l];
						}
						sumi += sc[c * 8 + g * 2 + half] * s;
					}
			acc = fmaf(d, (float)sumi, acc);
		}
	}
	return acc + acc_m;
}

/*
 * dot_f32_q4_K (quant.c:198-251): 8 lanes, lane l the elements k = l mod 8
 * in increasing k, each weight fl(fl(d * sc) * q) - fl(dmin * m), then an
 * FMA with x; the lane tree.  dot_f32_q6_K (quant.c:298-418): weights
 * fl((q - 32) * fl(d * sc)), FMAs in the same lane order.
 */
static float dot_q4_K_f32(const float *x, const uint8_t *row, size_t n)
{
	float acc[LANES] = {0};
	for (size_t i = 0; i < n / QKK; i++) {
		const uint8_t *b = row + i * 144;
		const float d = h2f(rd16(b)), dmin = h2f(rd16(b + 2));
		const uint8_t *q = b + 16;
		const float *xb = x + i * QKK;
		for (int j = 0; j < 4; j++) {
			int s1, m1, s2, m2;
			scale_min_k4(2 * j, b + 4, &s1, &m1);
			scale_min_k4(2 * j + 1, b + 4, &s2, &m2);
			const float d1 = d * (float)s1, n1 = dmin * (float)m1;
			const float d2 = d * (float)s2, n2 = dmin * (float)m2;
			for (int g = 0; g < 32; g += LANES)
				for (int l = 0; l < LANES; l++) {
					float v = d1 * (float)(q[j * 32 + g + l] & 0xF);
					v = v - n1;
					acc[l] = fmaf(v, xb[j * 64 + g + l], acc[l]);
				}
			for (int g = 0; g < 32; g += LANES)
				for (int l = 0; l < LANES; l++) {
					float v = d2 * (float)(q[j * 32 + g + l] >> 4);
					v = v - n2;
					acc[l] = fmaf(v, xb[j * 64 + 32 + g + l], acc[l]);
				}
		}
	}
	return lane_sum(acc);
}

static float dot_q6_K_f32(const float *x, const uint8_t *row, size_t n)
{
	float acc[LANES] = {0};
	for (size_t i = 0; i < n / QKK; i++) {
		const uint8_t *b = row + i * 210;
		const uint8_t *ql0 = b, *qh0 = b + 128;
		const int8_t *sc = (const int8_t *)(b + 192);
		const float d = h2f(rd16(b + 208));
		const float *xb = x + i * QKK;
		for (int c = 0; c < 2; c++) {
			const uint8_t *ql = ql0 + c * 64, *qh = qh0 + c * 32;
			for (int g = 0; g < 4; g++) {
				float tmp[32];
				for (int l = 0; l < 32; l++) {
					const int lo = g & 1 ? ql[l + 32] : ql[l];
					tmp[l] = (float)(((g < 2 ? lo & 0xF : lo >> 4) |
							  (((qh[l] >> (2 * g)) & 3) << 4)) -
							 32);
				}
				for (int half = 0; half < 2; half++) {
					const float vs = d * (float)sc[c * 8 + g * 2 + half];
					for (int u = 0; u < 16; u += LANES)
						for (int l = 0; l < LANES; l++) {
							const float vt = tmp[half * 16 + u + l] * vs;
							acc[l] = fmaf(vt, xb[c * 128 + g * 32 + half * 16 + u + l],
								      acc[l]);
						}
				}
			}
		}
	}
	return lane_sum(acc);
}

/* dequant_row_q4_K / q6_K (quant.c:420-531) */
static void dequant_kquant(const uint8_t *row, int wtype, float *dst, size_t n)
{
	for (size_t i = 0; i < n / QKK; i++) {
		float *o = dst + i * QKK;
		if (wtype == ORC_Q4_K) {
			const uint8_t *b = row + i * 144;
			const float d = h2f(rd16(b)), dmin = h2f(rd16(b + 2));
			for (int j = 0; j < 4; j++) {
				int s1, m1, s2, m2;
				scale_min_k4(2 * j, b + 4, &s1, &m1);
				scale_min_k4(2 * j + 1, b + 4, &s2, &m2);
				const float d1 = d * (float)s1, n1 = dmin * (float)m1;
				const float d2 = d * (float)s2, n2 = dmin * (float)m2;
				for (int k = 0; k < 32; k++) {
					float v = d1 * (float)(b[16 + j * 32 + k] & 0xF);
					o[j * 64 + k] = v - n1;
					v = d2 * (float)(b[16 + j * 32 + k] >> 4);
					o[j * 64 + 32 + k] = v - n2;
				}
			}
		} else {
			const uint8_t *b = row + i * 210;
			const int8_t *sc = (const int8_t *)(b + 192);
			const float d = h2f(rd16(b + 208));
			for (int c = 0; c < 2; c++) {
				const uint8_t *ql = b + c * 64, *qh = b + 128 + c * 32;
				for (int l = 0; l < 32; l++) {
					const int is = c * 8 + l / 16;
					const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
					const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
					const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
					const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
					/* d * scale * q: (d * scale) first, then * q (int -> float) */
					o[c * 128 + l + 0] = d * (float)sc[is + 0] * (float)q1;
					o[c * 128 + l + 32] = d * (float)sc[is + 2] * (float)q2;
					o[c * 128 + l + 64] = d * (float)sc[is + 4] * (float)q3;
					o[c * 128 + l + 96] = d * (float)sc[is + 6] * (float)q4;
				}
			}
		}
	}
}
