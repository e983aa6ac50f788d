/*
 * moe_qmm.hip - the dense quantized product for several tokens on the
 * gfx950 matrix cores, at fp32 accuracy:
 *   out[t][n] = add[t][n] (or add[n]) + sum_k x[t][k] * W[n][k]
 * with W N rows of K columns in Q8_0 or Q4_0 blocks (the reference's
 * tensor_mma_transposed_2x2 with a quantized right operand, matmul.c:451-462
 * -> 270-324, whose batched form tiles tokens and rows, matmul.c:145-165;
 * per element it is dot_f32_quant, quant.c:577-614).
 *
 * Exactness: a weight block is d * q with q small integers, exact in f16;
 * the block scale d stays out of the operand and is applied per block in
 * fp32.  A token block x (32 values) is scaled by a power of two 2^e (its
 * largest magnitude into [2^13, 2^14)) and split into two f16 parts,
 * hi = f16(x 2^e) and lo = f16(x 2^e - hi), which together hold x to ~22
 * bits.  One block of 16 tokens x 16 rows is then two
 * v_mfma_f32_16x16x32_f16 (hi, then lo, into a fresh accumulator: the
 * products q * hi and q * lo are exact in fp32), and
 *   acc += (d * 2^-e) * block
 * in fp32.  The result differs from an fp32 dot by the fp32 roundings of
 * other summation orders (~1e-7 relative), not by f16 rounding.
 *
 * Layouts.  The MFMA's K = 32 is split over the four 16-lane groups g of a
 * wave, eight values each; lane l holds token l % 16 (A) and row l % 16 (B)
 * of group l / 16, and the result D[token 4g + j][row l % 16] (j < 4).  The
 * values of group g are the block's elements 8g .. 8g+7 for Q8_0 (quant
 * bytes 8g.. of the block) and 4g .. 4g+3, 16+4g .. 16+4g+3 for Q4_0 (the
 * low and high nibbles of quant bytes 4g ..).  The tokens are split once
 * per call (k_qmm_split) into that order: xs[token][block] = hi groups 0-3
 * then lo groups 0-3 (8 f16 each, 128 bytes), tsc[block][token] = 2^-e,
 * tokens padded to a multiple of 16 with zeros.
 *
 * Work: a workgroup of four waves takes 16 rows and one tile of 16 tokens;
 * wave w the w-th quarter of K.  A wave loads all of its weights first
 * (Q4_0 five, Q8_0 seven dwords per lane and pair of blocks, the windows
 * aligned to 4 bytes), then walks its blocks with the next pair's token
 * operands in flight; the four quarters meet in LDS and are added in wave
 * order.
 *
 * Bound: HBM for a few tokens (the weights are read once per token tile;
 * the tokens, T * K * 4 bytes, come from L2).  Algorithmic bytes per call:
 * N * K/32 * block bytes + T*K*4 + T*N*4.
 */
#include "moe_device.h"
#include "moe_internal.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

#define QMM_ROWS 16
#define QMM_TOK 16
#define QMM_WAVES 4
#define QMM_MAX_PPW 16 /* pairs of blocks per wave: K up to 4096 */

/* ---------------------------------------------------------------------- */
/* token split                                                            */
/* ---------------------------------------------------------------------- */

/* thread (token t, block b, group g): the group's 8 values of x[t][32b..],
 * scaled by the block's 2^e, as hi and lo f16 */
template <int WT>
__global__ __launch_bounds__(256) void k_qmm_split(const float *__restrict__ x, int T, int TP,
						    int K, uint4 *__restrict__ xs,
						    float *__restrict__ tsc)
{
	const int nb = K / 32;
	const int i = blockIdx.x * 256 + threadIdx.x; /* TP * nb * 4 threads, a multiple of 64 */
	const int g = i & 3, b = (i >> 2) % nb, t = (i >> 2) / nb;
	float v[8];
	if (t < T) {
		const float *xb = x + (size_t)t * K + 32 * b;
		if (WT == 1) {
			const float4 p = ((const float4 *)(xb + 8 * g))[0];
			const float4 q = ((const float4 *)(xb + 8 * g))[1];
			v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
			v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
		} else {
			const float4 p = *(const float4 *)(xb + 4 * g);
			const float4 q = *(const float4 *)(xb + 16 + 4 * g);
			v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
			v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
		}
	} else {
#pragma unroll
		for (int k = 0; k < 8; k++)
			v[k] = 0.0f;
	}
	float m = 0.0f;
#pragma unroll
	for (int k = 0; k < 8; k++)
		m = fmaxf(m, fabsf(v[k]));
	m = fmaxf(m, __shfl_xor(m, 1, 4));
	m = fmaxf(m, __shfl_xor(m, 2, 4));
	/* 2^sh * m in [2^13, 2^14); a zero block keeps sh = 0 */
	int sh = 0;
	if (m > 0.0f) {
		const int ex = (int)((__builtin_bit_cast(u32, m) >> 23) & 0xffu) - 127;
		sh = 13 - ex;
		sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
	}
	const float s = __builtin_bit_cast(float, (u32)(sh + 127) << 23);
	half8_t hi, lo;
#pragma unroll
	for (int k = 0; k < 8; k++) {
		const float y = v[k] * s;
		const _Float16 h = (_Float16)y;
		hi[k] = h;
		lo[k] = (_Float16)(y - (float)h);
	}
	uint4 *o = xs + ((size_t)t * nb + b) * 8;
	o[g] = __builtin_bit_cast(uint4, hi);
	o[4 + g] = __builtin_bit_cast(uint4, lo);
	if (g == 0)
		tsc[(size_t)b * TP + t] = __builtin_bit_cast(float, (u32)(127 - sh) << 23);
}

/* ---------------------------------------------------------------------- */
/* the product                                                            */
/* ---------------------------------------------------------------------- */

__device__ static inline u32 qmm_ld(const uint8_t *p)
{
	return *(const u32 *)p;
}

/* two f16 (1024 + byte) from the bytes v_perm selects */
__device__ static inline u32 qmm_magic(u32 u, u32 sel)
{
	return __builtin_amdgcn_perm(0x64646464u, u, sel);
}

/* 8 bytes (w0 = bytes 0-3, w1 = 4-7), each biased by `off` - 1024, to 8 f16
 * byte - (off - 1024): exact small integers */
__device__ static inline half8_t qmm_half8(u32 w0, u32 w1, _Float16 off)
{
	typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
	const half2_t o2 = {off, off};
	const half2_t a = __builtin_bit_cast(half2_t, qmm_magic(w0, 0x04010400u)) - o2;
	const half2_t b = __builtin_bit_cast(half2_t, qmm_magic(w0, 0x04030402u)) - o2;
	const half2_t c = __builtin_bit_cast(half2_t, qmm_magic(w1, 0x04010400u)) - o2;
	const half2_t e = __builtin_bit_cast(half2_t, qmm_magic(w1, 0x04030402u)) - o2;
	half8_t r;
	r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
	r[4] = c[0]; r[5] = c[1]; r[6] = e[0]; r[7] = e[1];
	return r;
}

/* a lane's raw weights of one pair of blocks (2P, 2P+1) of its row */
template <int WT> struct qmm_pair;

template <> struct qmm_pair<2> { /* Q4_0: 36 bytes, 4-byte aligned */
	static constexpr int DW = 5;
	__device__ static inline void load(const uint8_t *base, int g, u32 (&w)[DW])
	{
		w[0] = qmm_ld(base + 4 * g);      /* even block: quant bytes 4g.. at +2+4g */
		w[1] = qmm_ld(base + 4 * g + 4);
		w[2] = qmm_ld(base + 20 + 4 * g); /* odd block: quant bytes 4g.. at +20+4g */
		w[3] = qmm_ld(base);              /* even scale: bytes 0-1 */
		w[4] = qmm_ld(base + 16);         /* odd scale: bytes 18-19 */
	}
	/* block h (0 even, 1 odd): the unscaled operand and d */
	__device__ static inline half8_t operand(const u32 (&w)[DW], int h, float &d)
	{
		const u32 q = h ? w[2] : __builtin_amdgcn_alignbit(w[1], w[0], 16);
		d = f16_bits_to_f32(h ? w[4] >> 16 : w[3] & 0xffffu);
		return qmm_half8(q & 0x0f0f0f0fu, (q >> 4) & 0x0f0f0f0fu, (_Float16)1032.0f);
	}
};

template <> struct qmm_pair<1> { /* Q8_0: 68 bytes, 4-byte aligned */
	static constexpr int DW = 7;
	__device__ static inline void load(const uint8_t *base, int g, u32 (&w)[DW])
	{
		w[0] = qmm_ld(base + 8 * g);      /* even block: quants 8g.. at +2+8g */
		w[1] = qmm_ld(base + 8 * g + 4);
		w[2] = qmm_ld(base + 8 * g + 8);
		w[3] = qmm_ld(base + 36 + 8 * g); /* odd block: quants 8g.. at +36+8g */
		w[4] = qmm_ld(base + 40 + 8 * g);
		w[5] = qmm_ld(base);              /* even scale: bytes 0-1 */
		w[6] = qmm_ld(base + 32);         /* odd scale: bytes 34-35 */
	}
	__device__ static inline half8_t operand(const u32 (&w)[DW], int h, float &d)
	{
		u32 q0, q1;
		if (h) {
			q0 = w[3];
			q1 = w[4];
		} else {
			q0 = __builtin_amdgcn_alignbit(w[1], w[0], 16);
			q1 = __builtin_amdgcn_alignbit(w[2], w[1], 16);
		}
		d = f16_bits_to_f32(h ? w[6] >> 16 : w[5] & 0xffffu);
		/* signed bytes: q ^ 0x80 = q + 128 */
		return qmm_half8(q0 ^ 0x80808080u, q1 ^ 0x80808080u, (_Float16)1152.0f);
	}
};

/*
 * Grid (ceil(N / 16), TP / 16), four waves.  PPW: pairs of blocks per wave
 * (K = 256 * PPW).
 */
template <int WT, int PPW>
__global__ __launch_bounds__(QMM_WAVES * WAVE) void k_qmm(
	const uint8_t *__restrict__ W, size_t rb, int N, int K, const uint4 *__restrict__ xs,
	const float *__restrict__ tsc, int T, int TP, const float *__restrict__ add, int add_rows,
	float *__restrict__ out)
{
	typedef qmm_pair<WT> P;
	constexpr int BB = WT == 1 ? 34 : 18;
	__shared__ floatx4 red[QMM_WAVES - 1][WAVE];
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int r = lane & 15, g = lane >> 4;
	const int n = blockIdx.x * QMM_ROWS + r, t0 = blockIdx.y * QMM_TOK;
	const int nb = K / 32, p0 = wave * PPW;
	/* rows past N repeat the last row (their results are not stored) */
	const uint8_t *row = W + (size_t)min(n, N - 1) * rb + (size_t)p0 * 2 * BB;

	u32 w[PPW][P::DW];
#pragma unroll
	for (int p = 0; p < PPW; p++)
		P::load(row + (size_t)p * 2 * BB, g, w[p]);

	/* token operands of pair p: hi and lo of both blocks, the scales of
	 * tokens 4g .. 4g+3 */
	const uint4 *xt = xs + ((size_t)(t0 + r) * nb) * 8 + g;
	auto ld_tok = [&](int p, uint4 (&a)[4], float4 (&ts)[2]) {
		const int b = 2 * (p0 + p);
		a[0] = xt[(size_t)b * 8];
		a[1] = xt[(size_t)b * 8 + 4];
		a[2] = xt[(size_t)(b + 1) * 8];
		a[3] = xt[(size_t)(b + 1) * 8 + 4];
		ts[0] = *(const float4 *)(tsc + (size_t)b * TP + t0 + 4 * g);
		ts[1] = *(const float4 *)(tsc + (size_t)(b + 1) * TP + t0 + 4 * g);
	};
	floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
	uint4 a[4], an[4];
	float4 ts[2], tn[2];
	ld_tok(0, a, ts);
#pragma unroll
	for (int p = 0; p < PPW; p++) {
		if (p + 1 < PPW)
			ld_tok(p + 1, an, tn);
#pragma unroll
		for (int h = 0; h < 2; h++) {
			float d;
			const half8_t bq = P::operand(w[p], h, d);
			const floatx4 z = {0.0f, 0.0f, 0.0f, 0.0f};
			floatx4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(
				__builtin_bit_cast(half8_t, a[2 * h]), bq, z, 0, 0, 0);
			blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(
				__builtin_bit_cast(half8_t, a[2 * h + 1]), bq, blk, 0, 0, 0);
			const float4 s = ts[h];
			acc[0] = __builtin_fmaf(d * s.x, blk[0], acc[0]);
			acc[1] = __builtin_fmaf(d * s.y, blk[1], acc[1]);
			acc[2] = __builtin_fmaf(d * s.z, blk[2], acc[2]);
			acc[3] = __builtin_fmaf(d * s.w, blk[3], acc[3]);
		}
		if (p + 1 < PPW) {
#pragma unroll
			for (int k = 0; k < 4; k++)
				a[k] = an[k];
			ts[0] = tn[0];
			ts[1] = tn[1];
		}
	}
	/* the quarters of K in wave order */
	if (wave > 0)
		red[wave - 1][lane] = acc;
	__syncthreads();
	if (wave > 0)
		return;
#pragma unroll
	for (int v = 0; v < QMM_WAVES - 1; v++) {
		const floatx4 o = red[v][lane];
		acc[0] += o[0];
		acc[1] += o[1];
		acc[2] += o[2];
		acc[3] += o[3];
	}
	if (n >= N)
		return;
#pragma unroll
	for (int j = 0; j < 4; j++) {
		const int t = t0 + 4 * g + j;
		if (t < T) {
			const size_t o = (size_t)t * N + n;
			out[o] = (add ? add[add_rows ? o : (size_t)n] : 0.0f) + acc[j];
		}
	}
}

/* ---------------------------------------------------------------------- */
/* host                                                                    */
/* ---------------------------------------------------------------------- */

extern "C" int moe_qmm_supported(int wtype, int K)
{
	return (wtype == 1 || wtype == 2) && K >= 256 && K % 256 == 0 &&
	       K / 256 <= QMM_MAX_PPW && ((K / 256) & (K / 256 - 1)) == 0;
}

extern "C" size_t moe_qmm_split_bytes(int T, int K)
{
	const size_t TP = (size_t)(T + QMM_TOK - 1) / QMM_TOK * QMM_TOK;
	return TP * (size_t)(K / 32) * 128 + (size_t)(K / 32) * TP * sizeof(float);
}

extern "C" int moe_launch_qmm_split(int wtype, const float *x, int T, int K, void *split,
				    void *stream)
{
	if (!moe_qmm_supported(wtype, K) || T < 1)
		return (int)hipErrorInvalidValue;
	const int TP = (T + QMM_TOK - 1) / QMM_TOK * QMM_TOK, nb = K / 32;
	uint4 *xs = (uint4 *)split;
	float *tsc = (float *)((uint8_t *)split + (size_t)TP * nb * 128);
	const int nthr = TP * nb * 4; /* a multiple of 256: TP % 16 == 0, nb % 8 == 0 */
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		hipLaunchKernelGGL(k_qmm_split<1>, dim3(nthr / 256), dim3(256), 0, s, x, T, TP, K, xs,
				   tsc);
	else
		hipLaunchKernelGGL(k_qmm_split<2>, dim3(nthr / 256), dim3(256), 0, s, x, T, TP, K, xs,
				   tsc);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_qmm(int wtype, const uint8_t *W, int N, int K, const void *split,
			      int T, const float *add, int add_rows, float *out, void *stream)
{
	if (!moe_qmm_supported(wtype, K) || N < 1 || T < 1 || N > 16 * 65535)
		return (int)hipErrorInvalidValue;
	const int TP = (T + QMM_TOK - 1) / QMM_TOK * QMM_TOK, nb = K / 32;
	if (TP / QMM_TOK > 65535)
		return (int)hipErrorInvalidValue;
	const uint4 *xs = (const uint4 *)split;
	const float *tsc = (const float *)((const uint8_t *)split + (size_t)TP * nb * 128);
	const size_t rb = (size_t)nb * (wtype == 1 ? 34 : 18);
	const dim3 grid((N + QMM_ROWS - 1) / QMM_ROWS, TP / QMM_TOK), blk(QMM_WAVES * WAVE);
	hipStream_t s = (hipStream_t)stream;
#define QMM(WTT, PP)                                                                        \
	if (wtype == WTT && K / 256 == PP) {                                                \
		hipLaunchKernelGGL((k_qmm<WTT, PP>), grid, blk, 0, s, W, rb, N, K, xs, tsc, T, TP, \
				   add, add_rows, out);                                     \
		return (int)hipGetLastError();                                              \
	}
	QMM(1, 1) QMM(1, 2) QMM(1, 4) QMM(1, 8) QMM(1, 16)
	QMM(2, 1) QMM(2, 2) QMM(2, 4) QMM(2, 8) QMM(2, 16)
#undef QMM
	return (int)hipErrorInvalidValue;
}
