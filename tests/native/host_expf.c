/*
 * Test helper: the device expf (llm.c_amd/csrc/moe_expf.h) evaluated on the
 * host, next to glibc's expf, so CPU tests can compare the two algorithms
 * exhaustively without a GPU.  Counts mismatching bit patterns in a range.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "moe_expf.h"

struct job {
	uint64_t b0, n, step;
	uint64_t bad;
	uint32_t first_bad;
};

static void *run(void *arg)
{
	struct job *j = arg;
	for (uint64_t i = 0; i < j->n; i += j->step) {
		uint32_t u = (uint32_t)(j->b0 + i);
		float x;
		memcpy(&x, &u, 4);
		float g = expf(x), m = moe_expf(x);
		uint32_t gu, mu;
		memcpy(&gu, &g, 4);
		memcpy(&mu, &m, 4);
		if (gu != mu && !(isnan(g) && isnan(m))) {
			if (!j->bad)
				j->first_bad = u;
			j->bad++;
		}
	}
	return NULL;
}

/* mismatches between glibc expf and moe_expf over bit patterns
 * b0, b0+step, ... below b0+n; *first_bad gets the first one found. */
uint64_t host_expf_mismatches(uint32_t b0, uint64_t n, uint64_t step, int nthreads,
			      uint32_t *first_bad)
{
	struct job jobs[64];
	pthread_t th[64];
	if (nthreads < 1)
		nthreads = 1;
	if (nthreads > 64)
		nthreads = 64;
	uint64_t per = (n / step + nthreads - 1) / nthreads * step;
	for (int t = 0; t < nthreads; t++) {
		uint64_t s = (uint64_t)t * per;
		jobs[t].b0 = b0 + s;
		jobs[t].n = s >= n ? 0 : (n - s < per ? n - s : per);
		jobs[t].step = step;
		jobs[t].bad = 0;
		jobs[t].first_bad = 0;
		pthread_create(&th[t], NULL, run, &jobs[t]);
	}
	uint64_t bad = 0;
	*first_bad = 0;
	for (int t = 0; t < nthreads; t++) {
		pthread_join(th[t], NULL);
		if (jobs[t].bad && !bad)
			*first_bad = jobs[t].first_bad;
		bad += jobs[t].bad;
	}
	return bad;
}

/* moe_expf over an array (host evaluation). */
void host_moe_expf(const float *in, float *out, uint64_t n)
{
	for (uint64_t i = 0; i < n; i++)
		out[i] = moe_expf(in[i]);
}
