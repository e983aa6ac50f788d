/*
 * Seeded synthetic MoE layer inputs in GGUF block layout (see moe_synth.h).
 *
 * Quantizers follow the reference:
 *   quantize_row_q8_0   quant.c:62-78 (fp16 scale via f32_to_f16, quant.c:46-60)
 *   quantize_q4_0_block test/quant.c:45-79
 * and, for the K-quant block formats (quant.h:30-57), min/max quantizers of
 * this file's own (moe_quantize_q4_K / q6_K below).
 * Built with -ffp-contract=off so every product is rounded as written.
 */
#define _GNU_SOURCE
#include "moe_synth.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK 32
#define QKK 256

size_t moe_row_bytes(int wtype, size_t n)
{
	size_t nb = n / QK;
	if (wtype == 1)
		return nb * 34;
	if (wtype == 2)
		return nb * 18;
	if (wtype == 3)
		return n / QKK * 144;
	if (wtype == 5)
		return n / QKK * 210;
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

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void put16(uint8_t *p, uint16_t h)
{
	p[0] = (uint8_t)(h & 0xff);
	p[1] = (uint8_t)(h >> 8);
}

/*
 * Q4_K (144 bytes per 256 values: f16 d, f16 dmin, 12 bytes of 6-bit
 * sub-block scales and mins, 128 bytes of nibbles; quant.h:30-36).  Each
 * sub-block of 32 spans [lo, hi] with lo = min(0, min x): scale (hi - lo)/15
 * and min -lo, both as 6-bit multiples of the super-block's d = max scale/63
 * and dmin = max min/63 (f16, nearest even); values q = clamp(round((x + m) /
 * s), 0, 15).  The packing is the one get_scale_min_k4 (quant.h:63-73)
 * reads: bytes 0-3 scales 0-3 (6 bits) with scales 4-7's top 2 bits above,
 * bytes 4-7 mins 0-3 likewise, bytes 8-11 scales 4-7's low nibble with mins
 * 4-7's low nibble above; nibble byte j*32+k holds value j*64+k below and
 * j*64+32+k above.
 */
void moe_quantize_q4_K(const float *x, void *blocks, size_t n)
{
	uint8_t *out = blocks;
	for (size_t b = 0; b < n / QKK; b++) {
		const float *xb = &x[b * QKK];
		uint8_t *blk = out + b * 144;
		float sub_s[8], sub_m[8], smax = 0, mmax = 0;
		for (int j = 0; j < 8; j++) {
			float lo = 0, hi = -INFINITY;
			for (int k = 0; k < 32; k++) {
				float v = xb[j * 32 + k];
				lo = v < lo ? v : lo;
				hi = v > hi ? v : hi;
			}
			sub_s[j] = (hi - lo) / 15.0f;
			sub_m[j] = -lo;
			smax = sub_s[j] > smax ? sub_s[j] : smax;
			mmax = sub_m[j] > mmax ? sub_m[j] : mmax;
		}
		uint16_t hd = moe_f32_to_f16_rne(smax / 63.0f), hm = moe_f32_to_f16_rne(mmax / 63.0f);
		float d = moe_f16_to_f32(hd), dmin = moe_f16_to_f32(hm);
		put16(blk, hd);
		put16(blk + 2, hm);
		int sc[8], mn[8];
		for (int j = 0; j < 8; j++) {
			sc[j] = d > 0 ? clampi((int)roundf(sub_s[j] / d), 0, 63) : 0;
			mn[j] = dmin > 0 ? clampi((int)roundf(sub_m[j] / dmin), 0, 63) : 0;
		}
		uint8_t *p = blk + 4;
		for (int j = 0; j < 4; j++) {
			p[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
			p[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
			p[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
		}
		int q[QKK];
		for (int j = 0; j < 8; j++) {
			float s = d * (float)sc[j], m = dmin * (float)mn[j];
			for (int k = 0; k < 32; k++)
				q[j * 32 + k] = s > 0 ? clampi((int)roundf((xb[j * 32 + k] + m) / s), 0, 15) : 0;
		}
		uint8_t *qs = blk + 16;
		for (int j = 0; j < 4; j++)
			for (int k = 0; k < 32; k++)
				qs[j * 32 + k] = (uint8_t)(q[j * 64 + k] | (q[j * 64 + 32 + k] << 4));
	}
}

/*
 * Q6_K (210 bytes per 256 values: 128 bytes of low nibbles, 64 bytes of
 * 2-bit highs, 16 int8 sub-block scales, f16 d; quant.h:47-53).  Each
 * sub-block of 16 takes scale s = -v/32 for its value v of largest
 * magnitude (so v lands on -32 and scales carry either sign), stored as
 * int8 multiples of d = -(the s of largest magnitude)/128 (f16, nearest
 * even); values q = clamp(round(x / s), -32, 31), stored as q + 32.  Value
 * c*128 + g*32 + l (g = 0..3, l = 0..31) keeps its low nibble in byte
 * c*64 + (g & 1)*32 + l (below for g < 2, above otherwise) and its top two
 * bits in bits 2g..2g+1 of byte 128 + c*32 + l.
 */
void moe_quantize_q6_K(const float *x, void *blocks, size_t n)
{
	uint8_t *out = blocks;
	for (size_t b = 0; b < n / QKK; b++) {
		const float *xb = &x[b * QKK];
		uint8_t *blk = out + b * 210;
		float sub[16], smax = 0, sval = 0;
		for (int j = 0; j < 16; j++) {
			float amax = 0, v = 0;
			for (int k = 0; k < 16; k++) {
				float a = fabsf(xb[j * 16 + k]);
				if (a > amax) {
					amax = a;
					v = xb[j * 16 + k];
				}
			}
			sub[j] = -v / 32.0f;
			if (fabsf(sub[j]) > smax) {
				smax = fabsf(sub[j]);
				sval = sub[j];
			}
		}
		uint16_t hd = moe_f32_to_f16_rne(-sval / 128.0f);
		float d = moe_f16_to_f32(hd);
		memset(blk, 0, 192);
		int8_t *sc = (int8_t *)(blk + 192);
		for (int j = 0; j < 16; j++)
			sc[j] = (int8_t)(d != 0 ? clampi((int)roundf(sub[j] / d), -128, 127) : 0);
		put16(blk + 208, hd);
		for (int e = 0; e < QKK; e++) {
			float s = d * (float)sc[e / 16];
			int q = s != 0 ? clampi((int)roundf(xb[e] / s), -32, 31) : 0;
			int u = q + 32, c = e / 128, g = (e % 128) / 32, l = e % 32;
			uint8_t *lo = blk + c * 64 + (g & 1) * 32 + l;
			*lo |= (uint8_t)(g < 2 ? (u & 0xF) : ((u & 0xF) << 4));
			blk[128 + c * 32 + l] |= (uint8_t)((u >> 4) << (2 * g));
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
		else if (j->wtype == 2)
			moe_quantize_q4_0(row, j->blocks + r * rb, j->cols);
		else if (j->wtype == 3)
			moe_quantize_q4_K(row, j->blocks + r * rb, j->cols);
		else
			moe_quantize_q6_K(row, j->blocks + r * rb, j->cols);
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
