/*
 * kquant.hip - the dense product on K-quant matrices (Q4_K, Q6_K) for
 * gfx950, bit for bit the reference's default -DQ8_DOT build:
 *
 *   out[t][j] = add[t][j] (or add[j], or 0) + dot_q8_quant(q8(x[t]), W[j])
 *
 * tensor_mma_transposed_2x2 (matmul.c:270-324) quantizes every token to
 * Q8_K once (quantize_row_q8, quant.c:627-654) when K % 256 == 0, which a
 * K-quant matrix always satisfies, and takes dot_q4_K_q8_K / dot_q6_K_q8_K
 * (quant_avx2.h:8-209, equal bit for bit to quant_cpu.h:7-120) per output.
 * Those dots are exact integer sums per 256-value super-block followed by a
 * sequential fp32 accumulation over super-blocks, which this file keeps:
 *
 *   Q4_K: sumi = sum_j sc_j * sum(q4 * q8) over 8 sub-blocks of 32,
 *         msum = sum_j m_j * (bsum_{2j} + bsum_{2j+1});
 *         acc   = fma(yd * d,    sumi, acc)     (clang contracts
 *         acc_m = fma(-yd * dmin, msum, acc_m)   `acc += d * sumi`)
 *         dot = acc + acc_m
 *   Q6_K: sumi = sum_j sc_j * sum((q6 - 32) * q8) over 16 sub-blocks of 16,
 *         taken here as sum(q6u * q8) - 32 * bsum_j with q6u = q6 + 32 in
 *         0..63 (the same integer); acc = fma(yd * d, sumi, acc); dot = acc.
 *
 * The integer sums use v_dot4c_i32_i8 (four int8 products per lane per
 * instruction, exact in int32: |sumi| < 2^28).
 *
 * Geometry.  A thread owns one super-block of one row at a time (144 bytes
 * Q4_K, 210 bytes Q6_K at a 2-byte offset for odd blocks: the dwords from
 * the aligned address below are realigned with v_alignbyte).  A workgroup
 * (256 threads) takes R rows at a time, R = 256 / gcd(nb, 256) (nb = K/256
 * super-blocks a row) capped at 2048 blocks, so the R * nb blocks split
 * evenly over the threads; consecutive threads take consecutive blocks of
 * the row-major matrix.  Each block's integers and scale products go to LDS
 * and one thread per (row, token) then runs the sequential fp32
 * accumulation over the row's nb super-blocks.  Each workgroup quantizes
 * the tokens itself into LDS (Q8_K blocks padded to 68 dwords so the lanes
 * reading different blocks hit different banks), TT tokens at a time; the
 * weights of a block stay in registers for all TT tokens, and the next
 * block's weights load while the current one's dots run.  A Q6_K product
 * for one token instead streams the matrix through an LDS ring
 * (k_kq_stream below).
 *
 * Bound: HBM.  Algorithmic bytes per call: N * K/256 * (144 | 210) + T*K*4
 * (x) + T*N*4 (out) (+ T*N*4 with add).
 */
#include "moe_device.h"

#define KQ_THREADS 256
#define KQ_LDS_MAX 65536
#define KQ_QSTRIDE 68 /* dwords per staged Q8_K block: 64 + 4 of padding */
#define KQ_GRID 768

/* ------------------------------------------------------------------ */
/* Q8_K quantization of 256 values by one wave (quantize_row_q8)        */
/* ------------------------------------------------------------------ */

/*
 * Lane l holds values 4l..4l+3 of the block.  Returns the four quants
 * packed as bytes; *d the block scale, *bsum (lanes l % 4 == 0) the sum of
 * the 16 quants 4l..4l+15.  amax: the first value of largest magnitude
 * (strictly greater, scanning in order: NaNs never win, all-zero blocks
 * stay zero); iscale = -127 / mval, d = 1 / iscale, q = min(127,
 * (int)roundf(iscale * x)).
 */
__device__ static inline u32 q8k_block(float4 v, int lane, float *d, int *bsum)
{
	const float xv[4] = {v.x, v.y, v.z, v.w};
	float best = 0.0f, bv = 0.0f;
	int bi = 0x7fffffff;
#pragma unroll
	for (int j = 0; j < 4; j++) {
		const float a = fabsf(xv[j]);
		if (a > best) {
			best = a;
			bv = xv[j];
			bi = 4 * lane + j;
		}
	}
#pragma unroll
	for (int off = 32; off >= 1; off >>= 1) {
		const float ob = __shfl_xor(best, off, WAVE), ov = __shfl_xor(bv, off, WAVE);
		const int oi = __shfl_xor(bi, off, WAVE);
		if (ob > best || (ob == best && oi < bi)) {
			best = ob;
			bv = ov;
			bi = oi;
		}
	}
	u32 packed = 0;
	int s = 0;
	if (best == 0.0f) {
		*d = 0.0f;
	} else {
		const float iscale = -127.0f / bv;
		*d = 1.0f / iscale;
#pragma unroll
		for (int j = 0; j < 4; j++) {
			int q = (int)roundf(iscale * xv[j]);
			q = q < 127 ? q : 127;
			s += q;
			packed |= (u32)(q & 0xff) << (8 * j);
		}
	}
	s += __shfl_xor(s, 1, WAVE);
	s += __shfl_xor(s, 2, WAVE);
	*bsum = s;
	return packed;
}

/* Staged tokens: sq [TT][nb][KQ_QSTRIDE] dwords of quants, sd [TT][nb]
 * scales, sb [TT][nb][16] sums of 16. */
struct KqTok {
	int *sq;
	float *sd;
	int *sb;
};

/* one token held in LDS (xl, K floats) into its staged Q8_K blocks */
__device__ static inline void kq_stage_lds(const KqTok &st, const float *xl, int K)
{
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nb = K / 256;
	for (int b = wave; b < nb; b += (int)blockDim.x / WAVE) {
		const float4 v = ((const float4 *)(xl + (size_t)b * 256))[lane];
		float d;
		int bs;
		const u32 q = q8k_block(v, lane, &d, &bs);
		st.sq[b * KQ_QSTRIDE + lane] = (int)q;
		if (lane % 4 == 0)
			st.sb[b * 16 + lane / 4] = bs;
		if (lane == 0)
			st.sd[b] = d;
	}
}

__device__ static inline void kq_stage(const KqTok &st, const float *__restrict__ x, int K,
				       int t0, int TT)
{
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE, nb = K / 256;
	for (int b = wave; b < TT * nb; b += (int)blockDim.x / WAVE) {
		const int tok = b / nb, i = b % nb;
		const float4 v = ((const float4 *)(x + (size_t)(t0 + tok) * K + (size_t)i * 256))[lane];
		float d;
		int bs;
		const u32 q = q8k_block(v, lane, &d, &bs);
		st.sq[b * KQ_QSTRIDE + lane] = (int)q;
		if (lane % 4 == 0)
			st.sb[b * 16 + lane / 4] = bs;
		if (lane == 0)
			st.sd[b] = d;
	}
}

/* ------------------------------------------------------------------ */
/* one super-block's integer sums                                       */
/* ------------------------------------------------------------------ */

template <int WT> struct kq;

/* Q4_K: d, dmin (f16), scales[12], qs[128]: 36 dwords, 16-byte aligned */
template <> struct kq<3> {
	static constexpr int BYTES = 144, DW = 36;
	__device__ static inline void load(const uint8_t *p, u32 (&w)[DW]) { load_dwords<DW>(p, w); }
	/* q8: the block's 64 staged quant dwords, bs its 16 sums */
	__device__ static inline void sums(const u32 (&w)[DW], const int *q8, const int *bs,
					   float yd, float &dsc, int &sumi, float &dmn, int &msum)
	{
		dsc = yd * f16_bits_to_f32(w[0]);
		dmn = -yd * f16_bits_to_f32(w[0] >> 16);
		/* get_scale_min_k4 (quant.h:63-73) for sub-blocks 0..7, a byte each */
		const u32 s0 = w[1], s1 = w[2], s2 = w[3];
		const u32 sc_lo = s0 & 0x3f3f3f3fu, m_lo = s1 & 0x3f3f3f3fu;
		const u32 sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
		const u32 m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
		int si = 0, mi = 0;
#pragma unroll
		for (int j = 0; j < 4; j++) {
			const u32 scw = j < 2 ? sc_lo : sc_hi, mw = j < 2 ? m_lo : m_hi;
			const int sh = 16 * (j & 1);
			const int sa = (scw >> sh) & 0xff, sb = (scw >> (sh + 8)) & 0xff;
			const int ma = (mw >> sh) & 0xff, mb = (mw >> (sh + 8)) & 0xff;
			int lo = 0, hi = 0;
			const int4 *qa = (const int4 *)(q8 + 16 * j);
#pragma unroll
			for (int k = 0; k < 2; k++) {
				const int4 a = qa[k], b = qa[k + 2];
				const u32 *ws = &w[4 + 8 * j + 4 * k];
				lo = __builtin_amdgcn_sdot4((int)(ws[0] & 0x0f0f0f0fu), a.x, lo, false);
				lo = __builtin_amdgcn_sdot4((int)(ws[1] & 0x0f0f0f0fu), a.y, lo, false);
				lo = __builtin_amdgcn_sdot4((int)(ws[2] & 0x0f0f0f0fu), a.z, lo, false);
				lo = __builtin_amdgcn_sdot4((int)(ws[3] & 0x0f0f0f0fu), a.w, lo, false);
				hi = __builtin_amdgcn_sdot4((int)((ws[0] >> 4) & 0x0f0f0f0fu), b.x, hi, false);
				hi = __builtin_amdgcn_sdot4((int)((ws[1] >> 4) & 0x0f0f0f0fu), b.y, hi, false);
				hi = __builtin_amdgcn_sdot4((int)((ws[2] >> 4) & 0x0f0f0f0fu), b.z, hi, false);
				hi = __builtin_amdgcn_sdot4((int)((ws[3] >> 4) & 0x0f0f0f0fu), b.w, hi, false);
			}
			si += sa * lo + sb * hi;
			mi += ma * (bs[4 * j] + bs[4 * j + 1]) + mb * (bs[4 * j + 2] + bs[4 * j + 3]);
		}
		sumi = si;
		msum = mi;
	}
};

/* Q6_K: ql[128], qh[64], scales[16] (int8), d (f16): 210 bytes, 2-byte
 * aligned; loaded as 53 dwords from the 4-byte aligned address at or below
 * the block (the matrix buffer has slack past its end) and realigned */
template <> struct kq<5> {
	static constexpr int BYTES = 210, DW = 53;
	__device__ static inline void load(const uint8_t *p, u32 (&w)[DW])
	{
		const uintptr_t a = (uintptr_t)p;
		u32 raw[DW];
		load_dwords<DW>((const uint8_t *)(a & ~(uintptr_t)3), raw);
		const u32 sh = (u32)(a & 3);
#pragma unroll
		for (int k = 0; k < DW - 1; k++)
			w[k] = __builtin_amdgcn_alignbyte(raw[k + 1], raw[k], sh);
		w[DW - 1] = raw[DW - 1] >> (8 * sh);
	}
	__device__ static inline void sums(const u32 (&w)[DW], const int *q8, const int *bs,
					   float yd, float &dsc, int &sumi, float &dmn, int &msum)
	{
		dsc = yd * f16_bits_to_f32(w[52]);
		dmn = 0.0f;
		msum = 0;
		int si = 0;
#pragma unroll
		for (int c = 0; c < 2; c++)
#pragma unroll
			for (int g = 0; g < 4; g++)
#pragma unroll
				for (int half = 0; half < 2; half++) {
					const int4 a = *(const int4 *)(q8 + 32 * c + 8 * g + 4 * half);
					const int av[4] = {a.x, a.y, a.z, a.w};
					int s = 0;
#pragma unroll
					for (int m = 0; m < 4; m++) {
						const u32 lq = w[16 * c + (g & 1) * 8 + 4 * half + m];
						const u32 lo = g < 2 ? lq & 0x0f0f0f0fu : (lq >> 4) & 0x0f0f0f0fu;
						const u32 hq = w[32 + 8 * c + 4 * half + m];
						const u32 hi = ((hq >> (2 * g)) & 0x03030303u) << 4;
						s = __builtin_amdgcn_sdot4((int)(lo | hi), av[m], s, false);
					}
					const int j = 8 * c + 2 * g + half;
					const int sc = (int)(int8_t)((w[48 + j / 4] >> (8 * (j % 4))) & 0xff);
					si += sc * (s - 32 * bs[j]);
				}
		sumi = si;
	}
};

/* ------------------------------------------------------------------ */
/* the product                                                          */
/* ------------------------------------------------------------------ */

#define KQ_ARGS                                                                            \
	const uint8_t *__restrict__ W, int N, int K, int R, const float *__restrict__ x, int T, \
		int TT, const float *__restrict__ add, int add_rows, float *__restrict__ out

/* LDS words per staged token and per record array */
__host__ __device__ static inline int kq_tok_words(int nb) { return nb * KQ_QSTRIDE + nb + nb * 16; }
__host__ __device__ static inline int kq_rec_words(int R, int nb) { return R * (nb + 1); }

/*
 * x = rms_norm(a + b) * w of one token (b may be NULL) into LDS (xl, K <=
 * 4096 floats) with the model's row norm arithmetic (thread v adds the four
 * squares of float4 v of a + b, then of float4 v + 256, ...; the xor trees
 * of the four waves; their sums in order; sqrtf(sum / K + 1e-5f); then
 * (v / rms) * w), so the bits are the row norm kernel's (rmsnorm,
 * nn.c:8-31).  a + b also goes to h_out and x to x_out (either NULL).
 */
__device__ static void kq_norm_token(float *xl, const float *a, const float *b, const float *w,
				     int K, float *h_out, float *x_out)
{
	constexpr int NV = 4096 / 4 / KQ_THREADS;
	__shared__ float s_red[KQ_THREADS / WAVE];
	const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE, n4 = K / 4;
	float4 v[NV], u[NV], wv[NV];
#pragma unroll
	for (int k = 0; k < NV; k++) {
		const int c4 = tid + k * KQ_THREADS;
		if (c4 < n4) {
			v[k] = ((const float4 *)a)[c4];
			if (b)
				u[k] = ((const float4 *)b)[c4];
			wv[k] = ((const float4 *)w)[c4];
		}
	}
	float ss = 0.0f;
#pragma unroll
	for (int k = 0; k < NV; k++) {
		const int c4 = tid + k * KQ_THREADS;
		if (c4 < n4) {
			if (b) {
				v[k].x = v[k].x + u[k].x;
				v[k].y = v[k].y + u[k].y;
				v[k].z = v[k].z + u[k].z;
				v[k].w = v[k].w + u[k].w;
			}
			if (h_out)
				((float4 *)h_out)[c4] = v[k];
			const float q0 = v[k].x * v[k].x, q1 = v[k].y * v[k].y;
			const float q2 = v[k].z * v[k].z, q3 = v[k].w * v[k].w;
			ss = ss + q0;
			ss = ss + q1;
			ss = ss + q2;
			ss = ss + q3;
		}
	}
	for (int o = WAVE / 2; o > 0; o >>= 1)
		ss += __shfl_xor(ss, o, WAVE);
	if (lane == 0)
		s_red[wave] = ss;
	__syncthreads();
	float sum = 0.0f;
#pragma unroll
	for (int k = 0; k < KQ_THREADS / WAVE; k++)
		sum += s_red[k];
	const float rms = sqrtf(sum / (float)K + 1e-5f);
#pragma unroll
	for (int k = 0; k < NV; k++) {
		const int c4 = tid + k * KQ_THREADS;
		if (c4 < n4) {
			float4 x = v[k];
			x.x = (x.x / rms) * wv[k].x;
			x.y = (x.y / rms) * wv[k].y;
			x.z = (x.z / rms) * wv[k].z;
			x.w = (x.w / rms) * wv[k].w;
			((float4 *)xl)[c4] = x;
			if (x_out)
				((float4 *)x_out)[c4] = x;
		}
	}
}

/* NORM (one token): x is a, the token is rms_norm(a + xb) * nw, staged from
 * LDS after the records; workgroup 0 writes a + xb to h_out and the token
 * to x_out (either NULL) */
template <int WT, bool NORM>
__global__ __launch_bounds__(KQ_THREADS) void k_kq_gemv(KQ_ARGS, const float *__restrict__ xb,
							const float *__restrict__ nw, float *h_out,
							float *x_out)
{
	extern __shared__ __attribute__((aligned(16))) int kq_lds[];
	using B = kq<WT>;
	constexpr int NREC = WT == 3 ? 4 : 2;
	const int nb = K / 256, blocks = R * nb, tid = threadIdx.x;
	const int S = (blocks + KQ_THREADS - 1) / KQ_THREADS; /* items a thread takes per group */
	const int ngroups = (N + R - 1) / R;
	const size_t rb = (size_t)nb * B::BYTES;
	const int rstride = nb + 1, rw = kq_rec_words(R, nb);
	KqTok st;
	st.sq = kq_lds;
	st.sd = (float *)(kq_lds + TT * nb * KQ_QSTRIDE);
	st.sb = kq_lds + TT * nb * (KQ_QSTRIDE + 1);
	int *rec = kq_lds + TT * kq_tok_words(nb); /* [TT][NREC][rw] */

	if ((int)blockIdx.x >= ngroups)
		return; /* the whole workgroup: no barrier below waits for it */
	/* block b of group g: row g*R + b/nb (clamped for loads), super-block b%nb */
	auto bptr = [&](int g, int b) {
		const int row = min(g * R + b / nb, N - 1);
		return W + (size_t)row * rb + (size_t)(b % nb) * B::BYTES;
	};
	const int items = ((ngroups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x) * S;

	for (int t0 = 0; t0 < T; t0 += TT) {
		const int tt = min(TT, T - t0);
		__syncthreads(); /* the previous pass's readers of the staged tokens are done */
		if constexpr (NORM) {
			/* after the records, 16-byte aligned (float4 stores and reads) */
			float *xl = (float *)(kq_lds +
					      ((TT * (kq_tok_words(nb) + NREC * rw) + 3) & ~3));
			kq_norm_token(xl, x, xb, nw, K, blockIdx.x == 0 ? h_out : nullptr,
				      blockIdx.x == 0 ? x_out : nullptr);
			__syncthreads();
			kq_stage_lds(st, xl, K);
		} else {
			kq_stage(st, x, K, t0, tt);
		}
		__syncthreads();
		u32 wn[B::DW];
		{
			const int b0 = tid < blocks ? tid : 0;
			B::load(bptr(blockIdx.x, b0), wn);
		}
		for (int it = 0; it < items; it++) {
			const int g = blockIdx.x + (it / S) * gridDim.x, s = it % S;
			const int b = s * KQ_THREADS + tid;
			u32 w[B::DW];
#pragma unroll
			for (int k = 0; k < B::DW; k++)
				w[k] = wn[k];
			if (it + 1 < items) {
				const int g1 = blockIdx.x + ((it + 1) / S) * gridDim.x;
				const int b1 = ((it + 1) % S) * KQ_THREADS + tid;
				B::load(bptr(g1, b1 < blocks ? b1 : 0), wn);
			}
			if (b < blocks) {
				const int i = b % nb, slot = (b / nb) * rstride + i;
				for (int tok = 0; tok < tt; tok++) {
					const int q = tok * nb + i;
					float dsc, dmn;
					int sumi, msum;
					B::sums(w, st.sq + q * KQ_QSTRIDE, st.sb + q * 16, st.sd[q], dsc, sumi,
						dmn, msum);
					int *r = rec + tok * NREC * rw;
					((float *)r)[slot] = dsc;
					r[rw + slot] = sumi;
					if constexpr (NREC == 4) {
						((float *)r)[2 * rw + slot] = dmn;
						r[3 * rw + slot] = msum;
					}
				}
			}
			if (s != S - 1)
				continue;
			__syncthreads();
			/* the sequential accumulation over super-blocks, a thread per (row, token) */
			for (int u = tid; u < R * tt; u += KQ_THREADS) {
				const int rl = u % R, tok = u / R, row = g * R + rl;
				if (row >= N)
					continue;
				const int *r = rec + tok * NREC * rw + rl * rstride;
				float acc = 0.0f, acc_m = 0.0f;
				for (int i = 0; i < nb; i++) {
					acc = fmaf(((const float *)r)[i], (float)r[rw + i], acc);
					if constexpr (NREC == 4)
						acc_m = fmaf(((const float *)r)[2 * rw + i], (float)r[3 * rw + i],
							     acc_m);
				}
				const float dot = NREC == 4 ? acc + acc_m : acc;
				const size_t o = (size_t)(t0 + tok) * N + row;
				out[o] = (add ? add[add_rows ? o : (size_t)row] : 0.0f) + dot;
			}
			__syncthreads();
		}
	}
}

/*
 * Q6_K, one token, no add: the matrix streams through an LDS ring by LDS-DMA.
 * A tile is RT = 128 / nb rows (RT * nb <= 128 super-blocks, contiguous
 * bytes); each of the 8 waves moves its share of a tile with RG::PW
 * wave-wide global_load_lds_dwordx4 loads (1 KB each, the pieces past the
 * tile's end repeat its last one), NST - 1 tiles stay in flight, and a
 * workgroup (one per CU) takes tiles blockIdx.x, + gridDim.x, ...  Four
 * threads share a super-block, a quarter (64 values) each, and add their
 * exact integer sums across lanes; the row sums of the tile before (one
 * thread per row, nb sequential steps) run in waves 6-7 ahead of their
 * quarters.  Global loads inside the loop would make the compiler wait for
 * every DMA: the loop has none (the token is staged before it, the outputs
 * are stores).  Whole blocks per thread (128 of 256 threads busy) measured
 * 45 us for the Q6_K Mixtral lm_head against 34 for the register path:
 * the tile's dots, not the ring, were the bound (the ring alone streams at
 * ~6 TB/s).
 */
#define KQ_STHREADS 512
template <int WT> struct kq_ring;
template <> struct kq_ring<5> {
	static constexpr int PW = 4, NST = 4; /* 128 * 210 B = 26.3 KB a tile, 32 KB slots */
};
#define KQ_TB 128       /* super-blocks a tile holds at most */
#define KQ_STREAM_NB 32 /* super-blocks a row holds at most (K <= 8192) */
#define KQ_OBUF 1024    /* outputs a workgroup keeps in LDS until its last tile */

/* dwords at LDS address p (2-byte aligned): n of them, realigned.  The
 * aligned pointer is derived from p itself (not through an integer), so
 * the compiler keeps it in LDS: a flat load would also count in vmcnt and
 * make every read wait for the tiles in flight. */
template <int N>
__device__ static inline void lds_dwords_u16(const uint8_t *p, u32 (&w)[N])
{
	const u32 sh = (u32)((uintptr_t)p & 3);
	const u32 *q = (const u32 *)(p - sh);
	u32 raw[N + 1];
#pragma unroll
	for (int k = 0; k <= N; k++)
		raw[k] = q[k];
#pragma unroll
	for (int k = 0; k < N; k++)
		w[k] = __builtin_amdgcn_alignbyte(raw[k + 1], raw[k], sh);
}

/* quarter qt = (chunk c = qt / 2, half hf = qt % 2) of a Q6_K block in LDS:
 * values c*128 + g*32 + hf*16 + (0..15) for g = 0..3 */
__device__ static inline int q6k_quarter(const uint8_t *blk, int qt, const int *q8, const int *bs)
{
	const int c = qt >> 1, hf = qt & 1;
	u32 la[4], lb[4], hq[4];
	lds_dwords_u16<4>(blk + 64 * c + 16 * hf, la);      /* ql[l], l = 16hf .. 16hf+15 */
	lds_dwords_u16<4>(blk + 64 * c + 32 + 16 * hf, lb); /* ql[l + 32] */
	lds_dwords_u16<4>(blk + 128 + 32 * c + 16 * hf, hq); /* qh[l] */
	int si = 0;
#pragma unroll
	for (int g = 0; g < 4; g++) {
		const int4 a = *(const int4 *)(q8 + 32 * c + 8 * g + 4 * hf);
		const int av[4] = {a.x, a.y, a.z, a.w};
		int sm = 0;
#pragma unroll
		for (int m = 0; m < 4; m++) {
			const u32 lq = (g & 1) ? lb[m] : la[m];
			const u32 lo = g < 2 ? lq & 0x0f0f0f0fu : (lq >> 4) & 0x0f0f0f0fu;
			const u32 hi = ((hq[m] >> (2 * g)) & 0x03030303u) << 4;
			sm = __builtin_amdgcn_sdot4((int)(lo | hi), av[m], sm, false);
		}
		const int j = 8 * c + 2 * g + hf;
		const int sc = (int)(int8_t)blk[192 + j];
		si += sc * (sm - 32 * bs[j]);
	}
	return si;
}

template <int WT>
__global__ __launch_bounds__(KQ_STHREADS, 1) void k_kq_stream(const uint8_t *__restrict__ W, int N,
							      int K, const float *__restrict__ x,
							      float *__restrict__ out)
{
	constexpr int BYTES = kq<WT>::BYTES;
	using RG = kq_ring<WT>;
	constexpr int SLOT = RG::PW * 8192, NST = RG::NST;
	constexpr int NREC = WT == 3 ? 4 : 2;
	/* ring, staged token (up to KQ_STREAM_NB super-blocks) and two record
	 * sets of up to KQ_TB blocks and KQ_TB / 8 rows (nb >= 8): static, so
	 * the ~140-160 KB need no launch attribute */
	__shared__ __attribute__((aligned(16)))
	uint8_t kq_ring_lds[NST * SLOT + KQ_STREAM_NB * (KQ_QSTRIDE + 1 + 16) * 4 +
			    2 * NREC * (KQ_TB + KQ_TB / 8) * 4];
	/* the outputs: a store inside the loop would sit in this wave's vmcnt
	 * until acknowledged and hold back its next tile wait */
	__shared__ float obuf[KQ_OBUF];
	/* the DMA asm clobbers memory, after which the compiler would reload
	 * kernel arguments and the grid size with scalar loads and wait for
	 * them with lgkmcnt(0), which on gfx950 also waits for every LDS-DMA
	 * in flight (the ring ran at 3.5 TB/s instead of 6): they are pinned
	 * in registers once here */
	int G = (int)gridDim.x;
	asm volatile("" : "+s"(G));
	asm volatile("" : "+s"(N), "+s"(K), "+s"(W), "+s"(x), "+s"(out));
	const int nb = K / 256, RT = KQ_TB / nb, TB = RT * nb;
	const int tid = threadIdx.x, wave = tid / WAVE;
	const size_t rb = (size_t)nb * BYTES;
	const int ntiles = (N + RT - 1) / RT;
	const int mine = ((int)blockIdx.x < ntiles) ? (ntiles - (int)blockIdx.x + G - 1) / G : 0;
	uint8_t *ring = kq_ring_lds;
	KqTok st;
	st.sq = (int *)(ring + NST * SLOT);
	st.sd = (float *)(st.sq + nb * KQ_QSTRIDE);
	st.sb = st.sq + nb * (KQ_QSTRIDE + 1);
	int *rec = st.sb + nb * 16; /* [2][NREC][TB + RT] */
	const int rw = TB + RT, rstride = nb + 1;
	const u32 ring0 = __builtin_amdgcn_readfirstlane(lds_addr(ring));

	if (mine == 0)
		return; /* the whole workgroup */
	auto issue = [&](int i) { /* the DMA loads of this workgroup's tile i into slot i % NST */
		const int t = blockIdx.x + i * G;
		const int rows = min(RT, N - t * RT);
		const int np = (int)((rows * rb + 15) / 16); /* 16-byte pieces (the buffer has slack) */
		const uint8_t *base = W + (size_t)t * RT * rb;
		const u32 sl = ring0 + (u32)((i % NST) * SLOT) + (u32)(wave * 1024);
#pragma unroll
		for (int k = 0; k < RG::PW; k++) {
			const int pc = min(k * KQ_STHREADS + tid, np - 1);
			dma_dwordx4(base, (u32)pc * 16u, sl + (u32)(k * 8192));
		}
	};
	/* the row sums of tile i (records set i & 1), thread u per row; the
	 * records are read 8 super-blocks at a time ahead of their FMAs (nb is
	 * a multiple of 8 here) */
	auto finish = [&](int i, int u) {
		const int t = blockIdx.x + i * G;
		if (u >= 0 && u < RT && t * RT + u < N) {
			const int *r = rec + (i & 1) * NREC * rw + u * rstride;
			float acc = 0.0f, acc_m = 0.0f;
			for (int j0 = 0; j0 < nb; j0 += 8) {
				float d[8], dm[8];
				int si[8], mi[8];
#pragma unroll
				for (int k = 0; k < 8; k++) {
					d[k] = ((const float *)r)[j0 + k];
					si[k] = r[rw + j0 + k];
					if constexpr (NREC == 4) {
						dm[k] = ((const float *)r)[2 * rw + j0 + k];
						mi[k] = r[3 * rw + j0 + k];
					}
				}
#pragma unroll
				for (int k = 0; k < 8; k++) {
					acc = fmaf(d[k], (float)si[k], acc);
					if constexpr (NREC == 4)
						acc_m = fmaf(dm[k], (float)mi[k], acc_m);
				}
			}
			const float v = 0.0f + (NREC == 4 ? acc + acc_m : acc);
			if ((i + 1) * RT <= KQ_OBUF)
				obuf[i * RT + u] = v;
			else
				out[(size_t)t * RT + u] = v; /* past the buffer (vocabularies above 256k) */
		}
	};

	/* the token comes by LDS-DMA too, into the last slot (its first tile is
	 * issued in iteration 0), ahead of the first tiles: waiting for it
	 * leaves the tiles in flight (a plain load here made the compiler
	 * wait for every tile, and the ring started empty) */
	{
		const u32 xs = ring0 + (u32)((NST - 1) * SLOT) + (u32)(wave * 1024);
		for (int k = 0; k < K / (4 * KQ_STHREADS); k++)
			dma_dwordx4(x, (u32)(k * KQ_STHREADS + tid) * 16u, xs + (u32)(k * 8192));
	}
	for (int i = 0; i < NST - 1; i++)
		if (i < mine)
			issue(i);
	if (mine >= NST - 1)
		wait_vm<RG::PW *(NST - 1)>();
	else
		wait_vm<0>();
	__syncthreads();
	kq_stage_lds(st, (const float *)(ring + (NST - 1) * SLOT), K);
	__syncthreads(); /* the slot is free again and the token staged */
	const int bk = tid >> 2, qt = tid & 3; /* super-block of the tile, quarter */
	for (int i = 0; i < mine; i++) {
		if (i + NST - 2 < mine)
			wait_vm<RG::PW *(NST - 2)>(); /* this wave's pieces of tile i are in LDS */
		else
			wait_vm<0>();
		__syncthreads(); /* every wave's pieces; tile i - 1's readers are done */
		if (i + NST - 1 < mine)
			issue(i + NST - 1); /* into the slot tile i - 1 used */
		if (i > 0)
			finish(i - 1, tid - (KQ_STHREADS - KQ_TB));
		const int t = blockIdx.x + i * G;
		const bool live = bk < TB && t * RT + bk / nb < N;
		const int j = bk % nb;
		const uint8_t *blk = ring + (i % NST) * SLOT + (live ? bk : 0) * BYTES;
		static_assert(WT == 5, "the ring instance is Q6_K's");
		int sumi = q6k_quarter(blk, qt, st.sq + j * KQ_QSTRIDE, st.sb + j * 16), msum = 0;
		sumi += __shfl_xor(sumi, 1, WAVE);
		sumi += __shfl_xor(sumi, 2, WAVE);
		if constexpr (NREC == 4) {
			msum += __shfl_xor(msum, 1, WAVE);
			msum += __shfl_xor(msum, 2, WAVE);
		}
		if (live && qt == 0) {
			const int slot = (bk / nb) * rstride + j;
			const float yd = st.sd[j];
			int *r = rec + (i & 1) * NREC * rw;
			const u32 hd = WT == 3 ? *(const u32 *)blk
					       : (u32)blk[208] | ((u32)blk[209] << 8);
			((float *)r)[slot] = yd * f16_bits_to_f32(hd);
			r[rw + slot] = sumi;
			if constexpr (NREC == 4) {
				((float *)r)[2 * rw + slot] = -yd * f16_bits_to_f32(hd >> 16);
				r[3 * rw + slot] = msum;
			}
		}
	}
	__syncthreads();
	finish(mine - 1, tid);
	__syncthreads();
	for (int o = tid; o < min(mine * RT, KQ_OBUF - KQ_OBUF % RT); o += KQ_STHREADS) {
		const int i = o / RT, u = o % RT, row = (blockIdx.x + i * G) * RT + u;
		if (row < N)
			out[row] = obuf[o];
	}
}

/* one wave per 256-value block: quantize_row_q8 into d[T][nb], qs[T][K],
 * bsums[T][nb][16] */
__global__ __launch_bounds__(KQ_THREADS) void k_q8k_quantize(const float *__restrict__ x, int T,
							     int K, float *__restrict__ d,
							     int8_t *__restrict__ qs,
							     int16_t *__restrict__ bsums)
{
	const int lane = threadIdx.x % WAVE;
	const int b = blockIdx.x * (KQ_THREADS / WAVE) + threadIdx.x / WAVE;
	if (b >= T * (K / 256))
		return;
	const float4 v = ((const float4 *)(x + (size_t)b * 256))[lane];
	float dd;
	int bs;
	const u32 q = q8k_block(v, lane, &dd, &bs);
	((u32 *)(qs + (size_t)b * 256))[lane] = q;
	if (lane % 4 == 0)
		bsums[(size_t)b * 16 + lane / 4] = (int16_t)bs;
	if (lane == 0)
		d[b] = dd;
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */

static int gcd_i(int a, int b)
{
	while (b) {
		const int t = a % b;
		a = b;
		b = t;
	}
	return a;
}

/* rows a workgroup takes at a time: R * nb a multiple of 256 where that
 * stays within 2048 blocks */
static int kq_rows(int nb)
{
	const int R = KQ_THREADS / gcd_i(nb, KQ_THREADS);
	if (R * nb <= 2048)
		return R;
	return max(1, KQ_THREADS / nb + (KQ_THREADS % nb != 0));
}

static size_t kq_lds_bytes(int wt, int K, int TT)
{
	const int nb = K / 256, R = kq_rows(nb);
	return (size_t)TT * (kq_tok_words(nb) + (wt == 3 ? 4 : 2) * kq_rec_words(R, nb)) * 4;
}

static int kq_tt(int wt, int K, int T)
{
	int tt = min(T, 8);
	while (tt > 1 && kq_lds_bytes(wt, K, tt) > KQ_LDS_MAX)
		tt--;
	return tt;
}

/* largest K the product takes: one token's LDS within KQ_LDS_MAX */
extern "C" int moe_kq_supported(int wtype, int K)
{
	if ((wtype != 3 && wtype != 5) || K < 256 || K % 256 || K > (1 << 20))
		return 0;
	return kq_lds_bytes(wtype, K, 1) <= KQ_LDS_MAX;
}

extern "C" int moe_kq_grid(int wtype, int K, int T)
{
	int dev = 0, ncu = 0, per = 0;
	if (!moe_kq_supported(wtype, K))
		return 0;
	const size_t lds = kq_lds_bytes(wtype, K, kq_tt(wtype, K, T));
	if (hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		return 0;
	const hipError_t e = wtype == 3 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(
						  &per, k_kq_gemv<3, false>, KQ_THREADS, lds)
					: hipOccupancyMaxActiveBlocksPerMultiprocessor(
						  &per, k_kq_gemv<5, false>, KQ_THREADS, lds);
	if (e != hipSuccess || per < 1)
		return 0;
	return per * ncu;
}

/* the streamed instance: one token, no add, K <= 128 * 256 with whole
 * 16-byte tiles */
/* Measured (Mixtral lm_head Q6_K 32000 x 4096 / OLMoE lm_head as Q4_K
 * 50304 x 2048, one token): the ring 29.4 / 20.5 us, the register path
 * 34 / 17.4 us.  Per tile the waves' dots and the barrier take ~1.5 us
 * against ~1.15 us of streaming, so the ring pays off only where the
 * register path's loads are costliest (Q6_K's 210-byte blocks at 2-byte
 * offsets): Q4_K keeps the register path. */
static int kq_stream_ok(int wt, int K, int T, const float *add)
{
	const int nb = K / 256;
	if (wt != 5 || T != 1 || add || nb > KQ_STREAM_NB || nb % 8 || K * 4 > 4 * 8192)
		return 0; /* the token must fit one ring slot */
	const int TB = (KQ_TB / nb) * nb;
	return (TB * (wt == 3 ? 144 : 210)) % 16 == 0;
}

extern "C" int moe_launch_kq_gemv(int wtype, const uint8_t *W, int N, int K, const float *x,
				  int T, const float *add, int add_rows, float *out, int nwg,
				  void *stream)
{
	if (!moe_kq_supported(wtype, K) || N < 1 || T < 1)
		return (int)hipErrorInvalidValue;
	if (kq_stream_ok(wtype, K, T, add)) {
		int dev = 0, ncu = 0;
		if (hipGetDevice(&dev) != hipSuccess ||
		    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) !=
			    hipSuccess)
			return (int)hipErrorInvalidValue;
		const int RT = KQ_TB / (K / 256), ntiles = (N + RT - 1) / RT;
		const dim3 grid(min(ntiles, ncu));
		hipStream_t s = (hipStream_t)stream;
		hipLaunchKernelGGL(k_kq_stream<5>, grid, dim3(KQ_STHREADS), 0, s, W, N, K, x, out);
		return (int)hipGetLastError();
	}
	const int nb = K / 256, R = kq_rows(nb), TT = kq_tt(wtype, K, T);
	const int ngroups = (N + R - 1) / R;
	const dim3 grid(min(ngroups, nwg > 0 ? nwg : KQ_GRID));
	const size_t lds = kq_lds_bytes(wtype, K, TT);
	hipStream_t s = (hipStream_t)stream;
	const float *nul = nullptr;
	float *nulw = nullptr;
	if (wtype == 3)
		hipLaunchKernelGGL((k_kq_gemv<3, false>), grid, dim3(KQ_THREADS), lds, s, W, N, K, R,
				   x, T, TT, add, add_rows, out, nul, nul, nulw, nulw);
	else
		hipLaunchKernelGGL((k_kq_gemv<5, false>), grid, dim3(KQ_THREADS), lds, s, W, N, K, R,
				   x, T, TT, add, add_rows, out, nul, nul, nulw, nulw);
	return (int)hipGetLastError();
}

extern "C" int moe_kq_norm_ok(int wtype, int K)
{
	return moe_kq_supported(wtype, K) && !kq_stream_ok(wtype, K, 1, NULL) && K <= 4096 &&
	       kq_lds_bytes(wtype, K, 1) + 16 + (size_t)K * 4 <= KQ_LDS_MAX;
}

extern "C" int moe_launch_kq_gemv_norm(int wtype, const uint8_t *W, int N, int K, const float *a,
				       const float *b, const float *w, float *h_out, float *x_out,
				       float *out, int nwg, void *stream)
{
	if (!moe_kq_norm_ok(wtype, K) || N < 1 || !a || !w)
		return (int)hipErrorInvalidValue;
	const int nb = K / 256, R = kq_rows(nb), TT = 1;
	const int ngroups = (N + R - 1) / R;
	const dim3 grid(min(ngroups, nwg > 0 ? nwg : KQ_GRID));
	const size_t lds = kq_lds_bytes(wtype, K, TT) + 16 + (size_t)K * 4;
	hipStream_t s = (hipStream_t)stream;
	const float *nul = nullptr;
	const int T = 1, add_rows = 0;
	if (wtype == 3)
		hipLaunchKernelGGL((k_kq_gemv<3, true>), grid, dim3(KQ_THREADS), lds, s, W, N, K, R,
				   a, T, TT, nul, add_rows, out, b, w, h_out, x_out);
	else
		hipLaunchKernelGGL((k_kq_gemv<5, true>), grid, dim3(KQ_THREADS), lds, s, W, N, K, R,
				   a, T, TT, nul, add_rows, out, b, w, h_out, x_out);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_q8k_quantize(const float *x, int T, int K, float *d, int8_t *qs,
				       int16_t *bsums, void *stream)
{
	if (T < 1 || K < 256 || K % 256)
		return (int)hipErrorInvalidValue;
	const int blocks = T * (K / 256);
	const int wpb = KQ_THREADS / WAVE;
	hipLaunchKernelGGL(k_q8k_quantize, dim3((blocks + wpb - 1) / wpb), dim3(KQ_THREADS), 0,
			   (hipStream_t)stream, x, T, K, d, qs, bsums);
	return (int)hipGetLastError();
}
