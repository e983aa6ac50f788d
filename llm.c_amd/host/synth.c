/*
 * Seeded synthetic MoE layer inputs in GGUF block layout (see moe_synth.h).
 *
 * Quantizers follow the reference:
 *   quantize_row_q8_0   quant.c:62-78 (fp16 scale via f32_to_f16, quant.c:46-60)
 *   quantize_q4_0_block test/quant.c:45-79
 * Built with -ffp-contract=off so every product is rounded as written.
 */
#define _GNU_SOURCE
#include "moe_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 32

size_t moe_row_bytes(int wtype, size_t n)
{
	size_t nb = n / QK;
	if (wtype == 1)
		return nb * 34;
	if (wtype == 2)
		return nb * 18;
	return 0;
}

/* splitmix64 output function (S. Vigna, public domain) used as a hash. */
static inline uint64_t mix64(uint64_t z)
{
	z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
	z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
	return z ^ (z >> 31);
}

static inline uint64_t stream_key(uint64_t seed, uint64_t stream)
{
	return mix64(seed ^ mix64(stream ^ 0xd1b54a32d192ed03ULL));
}

/* uniform in (0, 1] */
static inline double unif(uint64_t key, uint64_t i)
{
	uint64_t v = mix64(key + (i + 1) * 0x9e3779b97f4a7c15ULL);
	return (double)((v >> 11) + 1) * 0x1p-53;
}

/* Box-Muller: element 2p is r cos(2 pi u2), element 2p+1 is r sin(2 pi u2). */
static inline double normal_at(uint64_t key, uint64_t i)
{
	uint64_t p = i >> 1;
	double u1 = unif(key, 2 * p), u2 = unif(key, 2 * p + 1);
	double r = sqrt(-2.0 * log(u1));
	double a = 6.283185307179586476925286766559 * u2;
	return (i & 1) ? r * sin(a) : r * cos(a);
}

static void fill_normal(uint64_t key, uint64_t i0, float mean, float std,
			float *out, size_t n)
{
	for (size_t i = 0; i < n; i++)
		out[i] = (float)((double)mean + (double)std * normal_at(key, i0 + i));
}

struct normal_job {
	uint64_t key, i0;
	float mean, std;
	float *out;
	size_t n;
};

static void *normal_thread(void *arg)
{
	struct normal_job *j = arg;
	fill_normal(j->key, j->i0, j->mean, j->std, j->out, j->n);
	return NULL;
}

void moe_synth_normal(uint64_t seed, uint64_t stream, float mean, float std,
		      float *out, size_t n, int nthreads)
{
	uint64_t key = stream_key(seed, stream);
	if (nthreads < 2 || n < (1u << 16)) {
		fill_normal(key, 0, mean, std, out, n);
		return;
	}
	struct normal_job *jobs = calloc((size_t)nthreads, sizeof(*jobs));
	pthread_t *th = calloc((size_t)nthreads, sizeof(*th));
	size_t chunk = (n + nthreads - 1) / nthreads;
	for (int t = 0; t < nthreads; t++) {
		size_t s = (size_t)t * chunk < n ? (size_t)t * chunk : n;
		size_t e = s + chunk < n ? s + chunk : n;
		jobs[t] = (struct normal_job){key, s, mean, std, out + s, e - s};
		pthread_create(&th[t], NULL, normal_thread, &jobs[t]);
	}
	for (int t = 0; t < nthreads; t++)
		pthread_join(th[t], NULL);
	free(jobs);
	free(th);
}

uint16_t moe_f32_to_f16_rne(float f)
{
	uint32_t x;
	memcpy(&x, &f, 4);
	uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
	uint32_t ax = x & 0x7fffffffu;

	if (ax > 0x7f800000u) /* nan: keep top payload bits, force quiet */
		return sign | 0x7e00u | (uint16_t)((ax >> 13) & 0x3ffu);
	if (ax >= 0x477ff000u) /* >= 65520 rounds to infinity */
		return sign | 0x7c00u;
	if (ax < 0x38800000u) { /* below 2^-14: f16 subnormal or zero */
		float a;
		memcpy(&a, &ax, 4);
		return sign | (uint16_t)rintf(a * 0x1p24f);
	}
	uint32_t m = ax + 0xfffu + ((ax >> 13) & 1u); /* round to nearest even */
	m -= 112u << 23;                              /* rebias 127 -> 15 */
	return sign | (uint16_t)(m >> 13);
}

float moe_f16_to_f32(uint16_t h)
{
	uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
	uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, f;
	if (e == 0) {
		if (m == 0) {
			f = sign;
		} else {
			int sh = 0;
			while (!(m & 0x400)) {
				m <<= 1;
				sh++;
			}
			f = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ff) << 13);
		}
	} else if (e == 0x1f) {
		f = sign | 0x7f800000u | (m << 13);
	} else {
		f = sign | ((e + 112) << 23) | (m << 13);
	}
	float r;
	memcpy(&r, &f, 4);
	return r;
}

/* The truncating conversion of test/quant.c:53-66. */
static uint16_t f32_to_f16_trunc(float scale)
{
	uint32_t fs;
	memcpy(&fs, &scale, 4);
	uint32_t sign = (fs >> 16) & 0x8000u;
	uint32_t ex = (fs >> 23) & 0xffu;
	uint32_t mant = fs & 0x7fffffu;
	if (ex == 0)
		return (uint16_t)sign;
	if (ex == 0xff)
		return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0));
	int ne = (int)ex - 127 + 15;
	if (ne >= 0x1f)
		return (uint16_t)(sign | 0x7c00u);
	if (ne <= 0)
		return (uint16_t)sign;
	return (uint16_t)(sign | ((uint32_t)ne << 10) | (mant >> 13));
}

void moe_quantize_q8_0(const float *x, void *blocks, size_t n)
{
	uint8_t *out = blocks;
	for (size_t b = 0; b < n / QK; b++) {
		const float *xb = &x[b * QK];
		uint8_t *blk = out + b * 34;
		float amax = 0;
		for (int j = 0; j < QK; j++) {
			float a = fabsf(xb[j]);
			if (a > amax)
				amax = a;
		}
		float d = amax / 127.0f;
		float id = d != 0.0f ? 1.0f / d : 0.0f;
		uint16_t h = moe_f32_to_f16_rne(d);
		blk[0] = (uint8_t)(h & 0xff);
		blk[1] = (uint8_t)(h >> 8);
		for (int j = 0; j < QK; j++)
			blk[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
	}
}

void moe_quantize_q4_0(const float *x, void *blocks, size_t n)
{
	uint8_t *out = blocks;
	for (size_t b = 0; b < n / QK; b++) {
		const float *xb = &x[b * QK];
		uint8_t *blk = out + b * 18;
		float amax = 0.0f;
		for (int j = 0; j < QK; j++) {
			float a = fabsf(xb[j]);
			if (a > amax)
				amax = a;
		}
		float scale = amax / 7.0f;
		uint16_t h = f32_to_f16_trunc(scale);
		blk[0] = (uint8_t)(h & 0xff);
		blk[1] = (uint8_t)(h >> 8);
		float inv = scale > 0 ? 7.0f / amax : 0.0f;
		for (int j = 0; j < QK / 2; j++) {
			int lo = (int)roundf(xb[j] * inv) + 8;
			int hi = (int)roundf(xb[j + QK / 2] * inv) + 8;
			lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
			hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
			blk[2 + j] = (uint8_t)(lo | (hi << 4));
		}
	}
}

struct quant_job {
	uint64_t key;
	float std;
	int wtype;
	size_t r0, r1, cols;
	uint8_t *blocks;
};

static void *quant_thread(void *arg)
{
	struct quant_job *j = arg;
	float *row = malloc(j->cols * sizeof(float));
	size_t rb = moe_row_bytes(j->wtype, j->cols);
	for (size_t r = j->r0; r < j->r1; r++) {
		fill_normal(j->key, (uint64_t)r * j->cols, 0.0f, j->std, row, j->cols);
		if (j->wtype == 1)
			moe_quantize_q8_0(row, j->blocks + r * rb, j->cols);
		else
			moe_quantize_q4_0(row, j->blocks + r * rb, j->cols);
	}
	free(row);
	return NULL;
}

void moe_synth_quant_matrix(uint64_t seed, uint64_t stream, float std,
			    int wtype, size_t rows, size_t cols, void *blocks,
			    int nthreads)
{
	if (nthreads < 1)
		nthreads = 1;
	if ((size_t)nthreads > rows)
		nthreads = (int)rows;
	struct quant_job *jobs = calloc((size_t)nthreads, sizeof(*jobs));
	pthread_t *th = calloc((size_t)nthreads, sizeof(*th));
	size_t chunk = (rows + nthreads - 1) / nthreads;
	uint64_t key = stream_key(seed, stream);
	for (int t = 0; t < nthreads; t++) {
		size_t s = (size_t)t * chunk < rows ? (size_t)t * chunk : rows;
		size_t e = s + chunk < rows ? s + chunk : rows;
		jobs[t] = (struct quant_job){key, std, wtype, s, e, cols, blocks};
		if (nthreads == 1)
			quant_thread(&jobs[t]);
		else
			pthread_create(&th[t], NULL, quant_thread, &jobs[t]);
	}
	if (nthreads > 1)
		for (int t = 0; t < nthreads; t++)
			pthread_join(th[t], NULL);
	free(jobs);
	free(th);
}

uint64_t moe_stream_router(uint64_t layer) { return (layer << 32) | 0x100u; }
uint64_t moe_stream_bias(uint64_t layer) { return (layer << 32) | 0x101u; }
uint64_t moe_stream_gate(uint64_t layer, uint64_t e) { return (layer << 32) | (0x10000u + e); }
uint64_t moe_stream_up(uint64_t layer, uint64_t e) { return (layer << 32) | (0x20000u + e); }
uint64_t moe_stream_down(uint64_t layer, uint64_t e) { return (layer << 32) | (0x30000u + e); }
uint64_t moe_stream_input(uint64_t call) { return 0xa0000000u + call; }
uint64_t moe_stream_tensor(uint64_t layer, uint64_t kind) { return (layer << 32) | (0x400u + kind); }
