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
 * low and high nibbles of quant bytes 4g ..).
 *
 * Work: a workgroup of four waves takes 64 rows (16 a wave), one tile of 16
 * tokens and one stretch of QMM_PZ pairs of blocks (512 columns) of K.  It
 * first puts every load of its weights in flight (each wave its 16 rows:
 * Q4_0 five, Q8_0 seven dwords per lane and pair of blocks, windows aligned
 * to 4 bytes), then stages the 16 tokens' columns of its stretch in LDS,
 * split as above (hi and lo in [block][group][token] order, so a wave's
 * operand reads are 1 KB contiguous), so each token value is read once
 * per 64 rows.  With K longer than one stretch the stretches are
 * workgroups of their own (grid z), whose partial sums a second launch
 * adds in stretch order (k_qmm_reduce): deterministic, and enough
 * workgroups for the few-thousand-row projections.  (Adding them in the
 * product launch instead, by the last stretch of a tile to arrive, polling
 * epoch-tagged partials, measured 26.7 us against 22.8 us for the two
 * launches at 16 tokens x 6144 x 4096 Q4_0: the last arrivals' polls sit
 * in series behind the slowest stretch.)
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
#define QMM_PZ 8 /* pairs of blocks per workgroup: 512 columns of K; at 16
		  * the weights in flight take 256 VGPRs and one wave per SIMD
		  * fits (1.4x slower at 16 tokens x 6144 x 4096 Q4_0) */

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

/* the split of one token block: the 8 values of a lane group scaled by the
 * block's 2^e (the 4 groups of a block are lanes l, l ^ 16, l ^ 32, l ^ 48) */
__device__ static inline void qmm_split8(const float (&v)[8], half8_t &hi, half8_t &lo,
					 float &unscale)
{
	float m = 0.0f;
#pragma unroll
	for (int k = 0; k < 8; k++)
		m = fmaxf(m, fabsf(v[k]));
	m = fmaxf(m, __shfl_xor(m, 16, WAVE));
	m = fmaxf(m, __shfl_xor(m, 32, WAVE));
	/* 2^sh * m in [2^13, 2^14); a zero block keeps sh = 0 */
	int sh = 0;
	if (m > 0.0f) {
		const int ex = (int)((__builtin_bit_cast(u32, m) >> 23) & 0xffu) - 127;
		sh = 13 - ex;
		sh = sh > 100 ? 100 : sh < -100 ? -100 : sh;
	}
	const float s = __builtin_bit_cast(float, (u32)(sh + 127) << 23);
#pragma unroll
	for (int k = 0; k < 8; k++) {
		const float y = v[k] * s;
		const _Float16 h = (_Float16)y;
		hi[k] = h;
		lo[k] = (_Float16)(y - (float)h);
	}
	unscale = __builtin_bit_cast(float, (u32)(127 - sh) << 23);
}

/*
 * Grid (ceil(N / 64), ceil(T / 16), K / (64 PZ)), four waves.  PZ: pairs of
 * blocks per workgroup.  part (grid z > 1): [z][T][N] partial sums.
 */
template <int WT, int PZ>
__global__ __launch_bounds__(QMM_WAVES * WAVE) void k_qmm(
	const uint8_t *__restrict__ W, size_t rb, int N, int K, const float *__restrict__ x, int T,
	const float *__restrict__ add, int add_rows, float *__restrict__ out,
	float *__restrict__ part)
{
	typedef qmm_pair<WT> P;
	constexpr int BB = WT == 1 ? 34 : 18, NB = 2 * PZ;
	__shared__ uint4 s_hi[NB][4][QMM_TOK], s_lo[NB][4][QMM_TOK];
	/* read as float4: 16-byte aligned whatever else the LDS holds */
	__shared__ __attribute__((aligned(16))) float s_ts[NB][QMM_TOK];
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int r = lane & 15, g = lane >> 4;
	const int n = blockIdx.x * (QMM_WAVES * QMM_ROWS) + wave * QMM_ROWS + r;
	const int t0 = blockIdx.y * QMM_TOK, z = blockIdx.z;
	/* rows past N repeat the last row (their results are not stored) */
	const uint8_t *row = W + (size_t)min(n, N - 1) * rb + (size_t)z * PZ * 2 * BB;
	u32 w[PZ][P::DW];
#pragma unroll
	for (int p = 0; p < PZ; p++)
		P::load(row + (size_t)p * 2 * BB, g, w[p]);

	/* the tokens' blocks of this stretch, split into LDS: thread item i =
	 * (block, group, token), the token fastest, so a wave's stores are 1 KB
	 * contiguous (with the group fastest every lane of a wave hit the same
	 * banks); all of a thread's loads go out before any is used (a loop
	 * that waited for each made the staging eight round trips: 33 -> ? us
	 * for the Mixtral q/k/v product of 16 tokens) */
	constexpr int IT = QMM_TOK * NB * 4 / (QMM_WAVES * WAVE); /* items per thread */
	float v[IT][8];
#pragma unroll
	for (int u = 0; u < IT; u++) { /* every load first: one round trip */
		const int i = (int)threadIdx.x + u * QMM_WAVES * WAVE;
		const int t = i & 15, gg = (i >> 4) & 3, b = i >> 6;
		float4 p = {0.0f, 0.0f, 0.0f, 0.0f}, q = p;
		if (t0 + t < T) {
			const float *xb = x + (size_t)(t0 + t) * K + (size_t)(z * NB + b) * 32;
			p = WT == 1 ? ((const float4 *)(xb + 8 * gg))[0] : *(const float4 *)(xb + 4 * gg);
			q = WT == 1 ? ((const float4 *)(xb + 8 * gg))[1]
				    : *(const float4 *)(xb + 16 + 4 * gg);
		}
		v[u][0] = p.x; v[u][1] = p.y; v[u][2] = p.z; v[u][3] = p.w;
		v[u][4] = q.x; v[u][5] = q.y; v[u][6] = q.z; v[u][7] = q.w;
	}
#pragma unroll
	for (int u = 0; u < IT; u++) {
		const int i = (int)threadIdx.x + u * QMM_WAVES * WAVE;
		const int t = i & 15, gg = (i >> 4) & 3, b = i >> 6;
		half8_t hi, lo;
		float us;
		qmm_split8(v[u], hi, lo, us);
		s_hi[b][gg][t] = __builtin_bit_cast(uint4, hi);
		s_lo[b][gg][t] = __builtin_bit_cast(uint4, lo);
		if (gg == 0)
			s_ts[b][t] = us;
	}
	__syncthreads();

	floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
	for (int p = 0; p < PZ; p++) {
#pragma unroll
		for (int h = 0; h < 2; h++) {
			const int b = 2 * p + h;
			float d;
			const half8_t bq = P::operand(w[p], h, d);
			const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
			floatx4 blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(
				__builtin_bit_cast(half8_t, s_hi[b][g][r]), bq, zero, 0, 0, 0);
			blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(
				__builtin_bit_cast(half8_t, s_lo[b][g][r]), bq, blk, 0, 0, 0);
			const float4 s = *(const float4 *)&s_ts[b][4 * g];
			acc[0] = __builtin_fmaf(d * s.x, blk[0], acc[0]);
			acc[1] = __builtin_fmaf(d * s.y, blk[1], acc[1]);
			acc[2] = __builtin_fmaf(d * s.z, blk[2], acc[2]);
			acc[3] = __builtin_fmaf(d * s.w, blk[3], acc[3]);
		}
		/* one pair at a time: left to itself the scheduler issued every
		 * MFMA first and held all 64 results (256 AGPRs: one wave per
		 * SIMD) */
		__builtin_amdgcn_sched_barrier(0);
	}
	if (n >= N)
		return;
#pragma unroll
	for (int j = 0; j < 4; j++) {
		const int t = t0 + 4 * g + j;
		if (t >= T)
			continue;
		const size_t o = (size_t)t * N + n;
		if (gridDim.z == 1)
			out[o] = (add ? add[add_rows ? o : (size_t)n] : 0.0f) + acc[j];
		else
			part[(size_t)z * T * N + o] = acc[j];
	}
}

/* out = add + the stretches' partial sums, added in stretch order */
__global__ __launch_bounds__(256) void k_qmm_reduce(const float *__restrict__ part, int KS,
						     size_t TN, int N, const float *__restrict__ add,
						     int add_rows, float *__restrict__ out)
{
	const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
	if (o >= TN)
		return;
	float s = part[o];
	for (int k = 1; k < KS; k++)
		s += part[(size_t)k * TN + o];
	out[o] = (add ? add[add_rows ? o : o % (size_t)N] : 0.0f) + s;
}

/* ---------------------------------------------------------------------- */
/* host                                                                    */
/* ---------------------------------------------------------------------- */

static int qmm_pz(int K)
{
	return K / 64 < QMM_PZ ? K / 64 : QMM_PZ;
}

extern "C" int moe_qmm_supported(int wtype, int K)
{
	return (wtype == 1 || wtype == 2) && K >= 256 && K % 256 == 0 &&
	       (K <= 64 * QMM_PZ ? ((K / 256) & (K / 256 - 1)) == 0 : K % (64 * QMM_PZ) == 0);
}

/* the partial sums of a call with K longer than one stretch */
extern "C" size_t moe_qmm_work_bytes(int T, int N, int K)
{
	const int KS = K / (64 * qmm_pz(K));
	return KS > 1 ? (size_t)KS * T * N * sizeof(float) : 0;
}

/* stretches of 64 * PZ columns the product of K columns splits into (its
 * partial sums are KS slices of T * N floats when KS > 1) */
extern "C" int moe_qmm_stretches(int K)
{
	return K / (64 * qmm_pz(K));
}

/* parts_only: KS > 1 and only the partial sums, left for the caller to add
 * in stretch order (k_qmm_reduce's sum) */
static int launch_qmm(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
		      const float *add, int add_rows, float *out, void *work, bool parts_only,
		      void *stream)
{
	if (!moe_qmm_supported(wtype, K) || N < 1 || T < 1 || (size_t)T * N > 0xffffffffull)
		return (int)hipErrorInvalidValue;
	const int PZ = qmm_pz(K), KS = K / (64 * PZ);
	if ((T + QMM_TOK - 1) / QMM_TOK > 65535 || (KS > 1 && !work) || (parts_only && KS < 2))
		return (int)hipErrorInvalidValue;
	const size_t rb = (size_t)(K / 32) * (wtype == 1 ? 34 : 18);
	const dim3 grid((N + QMM_WAVES * QMM_ROWS - 1) / (QMM_WAVES * QMM_ROWS),
			(T + QMM_TOK - 1) / QMM_TOK, KS),
		blk(QMM_WAVES * WAVE);
	hipStream_t s = (hipStream_t)stream;
	float *part = (float *)work;
	bool done = false;
#define QMM(WTT, PP)                                                                        \
	if (!done && wtype == WTT && PZ == PP) {                                            \
		hipLaunchKernelGGL((k_qmm<WTT, PP>), grid, blk, 0, s, W, rb, N, K, x, T, add,   \
				   add_rows, out, part);                                    \
		done = true;                                                                \
	}
	QMM(1, 4) QMM(1, 8)
	QMM(2, 4) QMM(2, 8)
#undef QMM
	if (!done)
		return (int)hipErrorInvalidValue;
	if (KS > 1 && !parts_only) {
		const size_t TN = (size_t)T * N;
		hipLaunchKernelGGL(k_qmm_reduce, dim3((unsigned)((TN + 255) / 256)), dim3(256), 0, s,
				   part, KS, TN, N, add, add_rows, out);
	}
	return (int)hipGetLastError();
}

extern "C" int moe_launch_qmm(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
			      const float *add, int add_rows, float *out, void *work,
			      void *stream)
{
	return launch_qmm(wtype, W, N, K, x, T, add, add_rows, out, work, false, stream);
}

extern "C" int moe_launch_qmm_parts(int wtype, const uint8_t *W, int N, int K, const float *x,
				    int T, void *work, void *stream)
{
	return launch_qmm(wtype, W, N, K, x, T, NULL, 0, NULL, work, true, stream);
}
