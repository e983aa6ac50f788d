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
	return (n / QK) * (wtype == ORC_Q8_0 ? 34 : 18);
}

float orc_dot_quant(const float *x, const void *qrow, int wtype, size_t n)
{
	if (wtype == ORC_Q8_0)
		return dot_q8_0(x, qrow, n);
	if (wtype == ORC_Q4_0)
		return dot_q4_0(x, qrow, n);
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
};

/* thread tidx of nt takes output columns [tidx * ceil(N/nt), ...) of every
 * token (transposed_gemv_thread_fn, matmul.c:107-114) */
static void qmat_task(void *arg, int tidx, int nt)
{
	const struct qmat_job *w = arg;
	const size_t rb = row_bytes(w->wtype, w->K), chunk = (w->N + nt - 1) / nt;
	const size_t j0 = tidx * chunk, j1 = j0 + chunk < w->N ? j0 + chunk : w->N;
	for (size_t t = 0; t < w->T; t++)
		for (size_t j = j0; j < j1; j++) {
			float init = !w->add ? 0.0f
					     : w->add_len == w->N ? w->add[j] : w->add[t * w->N + j];
			w->out[t * w->N + j] =
				init + orc_dot_quant(&w->x[t * w->K], (const uint8_t *)w->q + j * rb,
						     w->wtype, w->K);
		}
}

void orc_qmat_mul(const float *x, size_t T, const void *q, int wtype, size_t N, size_t K,
		  const float *add, size_t add_len, float *out)
{
	struct qmat_job w = {x, q, wtype, T, N, K, add, add_len, out};
	orc_pool_run(qmat_task, &w, orc_pool_threads(T, K, N));
}

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
		} else {
			abort();
		}
	}
}

struct ffn_job {
	const float *x;
	const uint8_t *g8, *u8, *d8;
	int wtype;
	size_t E, EI;
	float *h, *out;
};

/* nn.c:455-478: thread tidx's chunk of gate/up rows, then SwiGLU in place */
static void ffn_gateup_task(void *arg, int tidx, int nt)
{
	const struct ffn_job *w = arg;
	const size_t rb_in = row_bytes(w->wtype, w->E), chunk = (w->EI + nt - 1) / nt;
	const size_t j0 = tidx * chunk, j1 = j0 + chunk < w->EI ? j0 + chunk : w->EI;
	for (size_t j = j0; j < j1; j++) {
		float g = orc_dot_quant(w->x, w->g8 + j * rb_in, w->wtype, w->E);
		float u = orc_dot_quant(w->x, w->u8 + j * rb_in, w->wtype, w->E);
		w->h[j] = (g / (1.0f + expf(-g))) * u;
	}
}

/* nn.c:483-492: after the barrier, thread tidx's chunk of down rows */
static void ffn_down_task(void *arg, int tidx, int nt)
{
	const struct ffn_job *w = arg;
	const size_t rb_mid = row_bytes(w->wtype, w->EI), chunk = (w->E + nt - 1) / nt;
	const size_t i0 = tidx * chunk, i1 = i0 + chunk < w->E ? i0 + chunk : w->E;
	for (size_t i = i0; i < i1; i++)
		w->out[i] = orc_dot_quant(w->h, w->d8 + i * rb_mid, w->wtype, w->EI);
}

void orc_fused_ffn(const float *x, const void *gate, const void *up,
		   const void *down, int wtype, size_t E, size_t EI,
		   float *h, float *out)
{
	struct ffn_job w = {x, gate, up, down, wtype, E, EI, h, out};
	/* fused_ffn_silu's thread_pool_run(.., 1, k, inter) (nn.c:534) */
	const int nt = orc_pool_threads(1, E, EI);
	orc_pool_run(ffn_gateup_task, &w, nt);
	orc_pool_run(ffn_down_task, &w, nt);
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
