/*
 * kq_moe.hip - the MoE FFN's expert products on K-quant experts (Q4_K /
 * Q6_K, gate/up and down types chosen apart, as a Q4_K_M file mixes them),
 * bit for bit the reference's fused_ffn_silu (nn.c:449-539) in its default
 * -DQ8_DOT build:
 *
 *   k_kq_gateup  per (token, slot) pair p and rows j of expert ids[p]:
 *                g, u = dot_q8_quant(q8(x_t), gate/up row j) (the Q8_K
 *                integer dots of kquant.hip, the token quantized by each
 *                workgroup), h[p][j] = (g / (1 + expf(-g))) * u
 *                (nn.c:455-478; expf is glibc's, moe_expf.h)
 *   k_kq_down    y[p][i] = dot_f32_quant(h[p], down row i) (nn.c:483-492):
 *                the fp32 K-quant dot of quant.c:198-418 in its own order:
 *                accumulator l (of 8) takes elements l, l + 8, ... in
 *                increasing order with FMA, each weight fl(fl(d * sc) * q)
 *                - fl(dmin * m) (Q4_K) or fl((q - 32) * fl(d * sc)) (Q6_K),
 *                then the tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
 *
 * The combine (k_combine, y / (1/w) added in slot order) completes
 * olmoe.c:355-406 / llama.c:407-456, so the layer's outputs equal the
 * reference's bit for bit.
 *
 * Geometry.  k_kq_gateup: a workgroup per (pair, R = 128 / nb rows), a
 * thread per super-block of the R gate and R up rows (nb = E / 256 a row),
 * the block sums meet in LDS and a thread per row runs the sequential fp32
 * steps.  k_kq_down: 8 lanes per down row (lane l holds accumulator l), 32
 * rows per workgroup; the rows' super-blocks come through LDS in chunks of
 * KD_CB (contiguous runs, coalesced) with the matching KD_CB * 256 values
 * of h[p].
 *
 * Bound: HBM.  Algorithmic bytes per call: per pair, 2 * EI rows of E
 * columns and E rows of EI columns in their block types, plus x and h.
 */
#include "moe_device.h"

#define KG_THREADS 256
#define KD_THREADS 256
#define KD_ROWS 32 /* down rows a workgroup takes: 8 lanes each */
#define KD_CB 4    /* super-blocks of every row a chunk stages */

template <int WT> struct kqb;
template <> struct kqb<3> {
	static constexpr int BYTES = 144;
};
template <> struct kqb<5> {
	static constexpr int BYTES = 210;
};

/* ------------------------------------------------------------------ */
/* Q8_K of one token and the integer sums of one super-block            */
/* ------------------------------------------------------------------ */

/* quantize_row_q8 (quant.c:627-654) of 256 values, lane l holding 4l..4l+3
 * (the same steps as kquant.hip's) */
__device__ static inline u32 kg_q8k(float4 v, int lane, float *d, int *bsum)
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

/* dwords of a block at a 2-byte aligned global address: n, realigned (the
 * buffer is readable MOE_WEIGHT_SLACK bytes past its last block) */
template <int N>
__device__ static inline void kg_load(const uint8_t *p, u32 (&w)[N])
{
	const u32 sh = (u32)((uintptr_t)p & 3);
	u32 raw[N + 1];
	load_dwords<N + 1>(p - sh, raw);
#pragma unroll
	for (int k = 0; k < N; k++)
		w[k] = __builtin_amdgcn_alignbyte(raw[k + 1], raw[k], sh);
}

/* Q4_K block (36 dwords) against the staged Q8_K block q8 (64 dwords, its
 * 16 sums bs): sumi and msum, and the scale products with yd */
__device__ static inline void kg_q4k(const u32 (&w)[36], const int *q8, const int *bs, float yd,
				     float &dsc, int &sumi, float &dmn, int &msum)
{
	dsc = yd * f16_bits_to_f32(w[0]);
	dmn = -yd * f16_bits_to_f32(w[0] >> 16);
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
#pragma unroll
		for (int k = 0; k < 8; k++) {
			lo = __builtin_amdgcn_sdot4((int)(w[4 + 8 * j + k] & 0x0f0f0f0fu), q8[16 * j + k],
						    lo, false);
			hi = __builtin_amdgcn_sdot4((int)((w[4 + 8 * j + k] >> 4) & 0x0f0f0f0fu),
						    q8[16 * j + 8 + k], hi, false);
		}
		si += sa * lo + sb * hi;
		mi += ma * (bs[4 * j] + bs[4 * j + 1]) + mb * (bs[4 * j + 2] + bs[4 * j + 3]);
	}
	sumi = si;
	msum = mi;
}

/* Q6_K block (53 dwords): sumi with the q6 + 32 bytes, 32 * bsum taken off
 * per 16 values */
__device__ static inline void kg_q6k(const u32 (&w)[53], const int *q8, const int *bs, float yd,
				     float &dsc, int &sumi)
{
	dsc = yd * f16_bits_to_f32(w[52]);
	int si = 0;
#pragma unroll
	for (int c = 0; c < 2; c++)
#pragma unroll
		for (int g = 0; g < 4; g++)
#pragma unroll
			for (int hf = 0; hf < 2; hf++) {
				int s = 0;
#pragma unroll
				for (int m = 0; m < 4; m++) {
					const u32 lq = w[16 * c + (g & 1) * 8 + 4 * hf + m];
					const u32 lo = g < 2 ? lq & 0x0f0f0f0fu : (lq >> 4) & 0x0f0f0f0fu;
					const u32 hi = ((w[32 + 8 * c + 4 * hf + m] >> (2 * g)) & 0x03030303u) << 4;
					s = __builtin_amdgcn_sdot4((int)(lo | hi), q8[32 * c + 8 * g + 4 * hf + m],
								   s, false);
				}
				const int j = 8 * c + 2 * g + hf;
				const int sc = (int)(int8_t)((w[48 + j / 4] >> (8 * (j % 4))) & 0xff);
				si += sc * (s - 32 * bs[j]);
			}
	sumi = si;
}

/* ------------------------------------------------------------------ */
/* gate/up                                                              */
/* ------------------------------------------------------------------ */

/*
 * Block b < 2 * R * nb of the workgroup: matrix b / (R * nb) (0 gate, 1 up),
 * row j0 + (b % (R * nb)) / nb, super-block b % nb.  Records (4 words: the
 * scale products and integer sums) per block in LDS, rows padded to nb + 1.
 */
template <int WT>
__global__ __launch_bounds__(KG_THREADS) void k_kq_gateup(
	const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, size_t gu_stride,
	const u32 *__restrict__ ids, const float *__restrict__ x, float *__restrict__ h, int K,
	int E, int EI, int R)
{
	/* the token's Q8_K blocks, rows padded by one int: a wave's lanes read
	 * up to 16 blocks at the same offset, which then fall in distinct banks
	 * (a 64-int stride put them all in one) */
	constexpr int QS = 65, BS = 17;
	__shared__ int s_q8[32 * QS]; /* E <= 8192 */
	__shared__ float s_d[32];
	__shared__ int s_bs[32 * BS];
	__shared__ int s_rec[4][512]; /* 2 R (nb + 1) <= 512 for R * nb <= 128 */
	constexpr int BY = kqb<WT>::BYTES, DW = WT == 3 ? 36 : 53;
	const int p = blockIdx.y, t = p / K, nb = E / 256;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int j0 = blockIdx.x * R, RB = R * nb, rs = nb + 1;
	const size_t rb = (size_t)nb * BY;
	const size_t eo = (size_t)ids[p] * gu_stride;

	/* the weights first (one block per thread), then the token */
	u32 w[DW];
	const int b = tid < 2 * RB ? tid : 0;
	const int mat = b / RB, rl = (b % RB) / nb, sb = b % nb;
	const int row = min(j0 + rl, EI - 1);
	const uint8_t *blk = (mat ? up : gate) + eo + (size_t)row * rb + (size_t)sb * BY;
	if constexpr (WT == 3)
		load_dwords<36>(blk, w);
	else
		kg_load<53>(blk, w);
	/* the wave's token blocks (nb <= 32: at most 8 a wave), loaded together */
	float4 xv[8];
#pragma unroll
	for (int u = 0; u < 8; u++) {
		const int i = wave + u * (KG_THREADS / WAVE);
		if (i < nb)
			xv[u] = ((const float4 *)(x + (size_t)t * E + (size_t)i * 256))[lane];
	}
#pragma unroll
	for (int u = 0; u < 8; u++) {
		const int i = wave + u * (KG_THREADS / WAVE);
		if (i >= nb)
			break;
		const float4 v = xv[u];
		float d;
		int bs;
		const u32 q = kg_q8k(v, lane, &d, &bs);
		s_q8[i * QS + lane] = (int)q;
		if (lane % 4 == 0)
			s_bs[i * BS + lane / 4] = bs;
		if (lane == 0)
			s_d[i] = d;
	}
	__syncthreads();
	if (tid < 2 * RB) {
		float dsc, dmn = 0.0f;
		int sumi, msum = 0;
		if constexpr (WT == 3)
			kg_q4k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi, dmn, msum);
		else
			kg_q6k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi);
		const int slot = (mat * R + rl) * rs + sb;
		((float *)s_rec[0])[slot] = dsc;
		s_rec[1][slot] = sumi;
		((float *)s_rec[2])[slot] = dmn;
		s_rec[3][slot] = msum;
	}
	__syncthreads();
	/* thread r < R: row j0 + r, the reference's sequential steps for gate and
	 * up (dot_q4_K_q8_K returns acc + acc_m, dot_q6_K_q8_K acc) */
	if (tid < R && j0 + tid < EI) {
		float v[2];
#pragma unroll
		for (int m = 0; m < 2; m++) {
			const int o = (m * R + tid) * rs;
			float acc = 0.0f, acc_m = 0.0f;
			for (int i = 0; i < nb; i++) {
				acc = fmaf(((const float *)s_rec[0])[o + i], (float)s_rec[1][o + i], acc);
				if constexpr (WT == 3)
					acc_m = fmaf(((const float *)s_rec[2])[o + i], (float)s_rec[3][o + i],
						     acc_m);
			}
			v[m] = WT == 3 ? acc + acc_m : acc;
		}
		const float g = v[0];
		h[(size_t)p * EI + j0 + tid] = (g / (1.0f + moe_expf(-g))) * v[1];
	}
}

/* ------------------------------------------------------------------ */
/* down                                                                 */
/* ------------------------------------------------------------------ */

/* accumulator l's part of one staged super-block (LDS) of a down row: the
 * elements l, l + 8, ... with h from LDS */
__device__ static inline void kd_q4k(const uint8_t *blk, const float *hb, int l, float &acc)
{
	/* as kd_q6k: every LDS read first, then the products in their order
	 * (element 64j + 32hi + 8m + l is step 8j + 4hi + m of the chain) */
	u32 sc[12], q[4][4];
	float hv[32];
	const u32 b0 = blk[0], b1 = blk[1], b2 = blk[2], b3 = blk[3];
#pragma unroll
	for (int i = 0; i < 12; i++)
		sc[i] = blk[4 + i];
#pragma unroll
	for (int j = 0; j < 4; j++)
#pragma unroll
		for (int m = 0; m < 4; m++)
			q[j][m] = blk[16 + 32 * j + l + 8 * m];
#pragma unroll
	for (int jj = 0; jj < 32; jj++)
		hv[jj] = hb[l + 8 * jj];
	const float d = f16_bits_to_f32(b0 | (b1 << 8));
	const float dmin = f16_bits_to_f32(b2 | (b3 << 8));
#pragma unroll
	for (int j = 0; j < 4; j++) {
		int s1, m1, s2, m2;
		/* get_scale_min_k4 (quant.h:63-73) for sub-blocks 2j, 2j + 1 */
		if (j < 2) {
			s1 = sc[2 * j] & 63;
			m1 = sc[2 * j + 4] & 63;
			s2 = sc[2 * j + 1] & 63;
			m2 = sc[2 * j + 5] & 63;
		} else {
			s1 = (sc[2 * j + 4] & 0xF) | ((sc[2 * j - 4] >> 6) << 4);
			m1 = (sc[2 * j + 4] >> 4) | ((sc[2 * j] >> 6) << 4);
			s2 = (sc[2 * j + 5] & 0xF) | ((sc[2 * j - 3] >> 6) << 4);
			m2 = (sc[2 * j + 5] >> 4) | ((sc[2 * j + 1] >> 6) << 4);
		}
		const float d1 = d * (float)s1, n1 = dmin * (float)m1;
		const float d2 = d * (float)s2, n2 = dmin * (float)m2;
#pragma unroll
		for (int m = 0; m < 4; m++) {
			float v = d1 * (float)(q[j][m] & 0xF);
			v = v - n1;
			acc = fmaf(v, hv[8 * j + m], acc);
		}
#pragma unroll
		for (int m = 0; m < 4; m++) {
			float v = d2 * (float)(q[j][m] >> 4);
			v = v - n2;
			acc = fmaf(v, hv[8 * j + 4 + m], acc);
		}
	}
}

__device__ static inline void kd_q6k(const uint8_t *blk, const float *hb, int l, float &acc)
{
	/* every LDS read of the super-block goes out before the first product
	 * (the grid holds one wave per SIMD, so nothing else hides a read's
	 * round trip); the products and their order are unchanged: element
	 * 128c + 32g + 16hf + 8m + l is step j = 16c + 4g + 2hf + m of the
	 * lane's chain */
	u32 ql[2][2][2][2], qh[2][2][2]; /* [c][hf][m][+32] and [c][hf][m] */
	int sc[16];
	float hv[32];
#pragma unroll
	for (int c = 0; c < 2; c++)
#pragma unroll
		for (int hf = 0; hf < 2; hf++)
#pragma unroll
			for (int m = 0; m < 2; m++) {
				const int e = 16 * hf + l + 8 * m;
				ql[c][hf][m][0] = blk[64 * c + e];
				ql[c][hf][m][1] = blk[64 * c + e + 32];
				qh[c][hf][m] = blk[128 + 32 * c + e];
			}
#pragma unroll
	for (int i = 0; i < 16; i++)
		sc[i] = ((const int8_t *)(blk + 192))[i];
	const u32 dlo = blk[208], dhi = blk[209];
#pragma unroll
	for (int jj = 0; jj < 32; jj++)
		hv[jj] = hb[l + 8 * jj];
	const float d = f16_bits_to_f32(dlo | (dhi << 8));
#pragma unroll
	for (int c = 0; c < 2; c++)
#pragma unroll
		for (int g = 0; g < 4; g++)
#pragma unroll
			for (int hf = 0; hf < 2; hf++) {
				const float vs = d * (float)sc[8 * c + 2 * g + hf];
#pragma unroll
				for (int m = 0; m < 2; m++) {
					const int lo = (int)ql[c][hf][m][g & 1];
					const int q = ((g < 2 ? lo & 0xF : lo >> 4) |
						       (((int)(qh[c][hf][m] >> (2 * g)) & 3) << 4)) -
						      32;
					const float vt = (float)q * vs;
					acc = fmaf(vt, hv[16 * c + 4 * g + 2 * hf + m], acc);
				}
			}
}

/*
 * Workgroup (row block r0 = blockIdx.x * KD_ROWS, pair p): wave w holds rows
 * r0 + 8w .. r0 + 8w + 7, lane 8k + l accumulator l of row r0 + 8w + k.
 * Each chunk of KD_CB super-blocks of all 32 rows goes to LDS (row r's run
 * is contiguous: KD_CB * BY bytes at row r, block c0), the 8 lanes of a row
 * then walk its blocks in order.
 */
template <int WT>
__global__ __launch_bounds__(KD_THREADS) void k_kq_down(const uint8_t *__restrict__ down,
						      size_t dn_stride, const u32 *__restrict__ ids,
						      const float *__restrict__ h, float *__restrict__ y,
						      int E, int EI)
{
	constexpr int BY = kqb<WT>::BYTES;
	constexpr int RUN = KD_CB * BY; /* bytes of one row's run (a multiple of 8) */
	__shared__ __attribute__((aligned(16))) float s_h[KD_CB * 256]; /* the chunk's h */
	__shared__ __attribute__((aligned(16))) uint8_t s_w[KD_ROWS * RUN];
	const int p = blockIdx.y, nb = EI / 256;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int l = lane & 7, rk = wave * 8 + lane / 8; /* row of the block */
	const int r0 = blockIdx.x * KD_ROWS;
	const size_t rb = (size_t)nb * BY;
	const uint8_t *base = down + (size_t)ids[p] * dn_stride;

	/* a chunk's 32 runs, 8 bytes a thread per step (runs are 2-byte aligned
	 * for Q6_K: dword pairs from the aligned address, realigned), and its h,
	 * into registers: every load goes out before any is stored (a loop that
	 * stored each before the next load waited ~13 round trips a chunk), and
	 * the next chunk's go out while this one's dots run */
	constexpr int NIT = (KD_ROWS * (RUN / 8) + KD_THREADS - 1) / KD_THREADS;
	constexpr int NH = (KD_CB * 64 + KD_THREADS - 1) / KD_THREADS;
	u32 v[NIT][3], shv[NIT];
	float4 hv[NH];
	auto load_chunk = [&](int c0) {
		const int run = min(KD_CB, nb - c0) * BY, cb = min(KD_CB, nb - c0);
#pragma unroll
		for (int it = 0; it < NIT; it++) {
			const int e = tid + it * KD_THREADS;
			const int r = e / (RUN / 8), o = 8 * (e % (RUN / 8));
			shv[it] = 0;
			if (e < KD_ROWS * (RUN / 8) && o < run) {
				const int row = min(r0 + r, E - 1);
				const uint8_t *src = base + (size_t)row * rb + (size_t)c0 * BY + o;
				const u32 sh = (u32)((uintptr_t)src & 3);
				const u32 *a = (const u32 *)(src - sh);
				v[it][0] = a[0];
				v[it][1] = a[1];
				v[it][2] = a[2];
				shv[it] = sh;
			}
		}
#pragma unroll
		for (int u = 0; u < NH; u++) {
			const int i = tid + u * KD_THREADS;
			if (i < cb * 64)
				hv[u] = ((const float4 *)(h + (size_t)p * EI + (size_t)c0 * 256))[i];
		}
	};
	float acc = 0.0f;
	load_chunk(0);
	for (int c0 = 0; c0 < nb; c0 += KD_CB) {
		const int cb = min(KD_CB, nb - c0);
		const int run = cb * BY;
		__syncthreads(); /* the previous chunk's readers are done */
#pragma unroll
		for (int u = 0; u < NH; u++) {
			const int i = tid + u * KD_THREADS;
			if (i < cb * 64)
				((float4 *)s_h)[i] = hv[u];
		}
#pragma unroll
		for (int it = 0; it < NIT; it++) {
			const int e = tid + it * KD_THREADS;
			const int r = e / (RUN / 8), o = 8 * (e % (RUN / 8));
			if (e < KD_ROWS * (RUN / 8) && o < run)
				*(uint2 *)(s_w + r * RUN + o) =
					make_uint2(__builtin_amdgcn_alignbyte(v[it][1], v[it][0], shv[it]),
						   __builtin_amdgcn_alignbyte(v[it][2], v[it][1], shv[it]));
		}
		__syncthreads();
		if (c0 + KD_CB < nb)
			load_chunk(c0 + KD_CB);
		for (int k = 0; k < cb; k++) {
			const uint8_t *blk = s_w + rk * RUN + k * BY;
			if constexpr (WT == 3)
				kd_q4k(blk, s_h + k * 256, l, acc);
			else
				kd_q6k(blk, s_h + k * 256, l, acc);
		}
	}
	/* vector_reduce_sum's tree: lanes l and l + 4, then l and l + 2, then 0
	 * and 1 (each add is one fp32 addition; which operand comes first does
	 * not change it) */
	acc = acc + __shfl_xor(acc, 4, 8);
	acc = acc + __shfl_xor(acc, 2, 8);
	acc = acc + __shfl_xor(acc, 1, 8);
	if (l == 0 && r0 + rk < E)
		y[(size_t)p * E + r0 + rk] = acc;
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */

extern "C" int moe_kq_layer_supported(int gt, int dt, size_t E, size_t EI)
{
	const int gk = gt == 3 || gt == 5, dk = dt == 3 || dt == 5;
	return gk && dk && E % 256 == 0 && EI % 256 == 0 && E <= 8192 && E / 256 <= 128 &&
	       EI <= 16384;
}

extern "C" int moe_launch_kq_gateup(int gt, const uint8_t *gate, const uint8_t *up,
				    size_t gu_stride, const u32 *ids, const float *x, float *h,
				    int P, int K, int E, int EI, void *stream)
{
	const int nb = E / 256, R = max(1, 128 / nb);
	const dim3 grid((EI + R - 1) / R, P);
	hipStream_t s = (hipStream_t)stream;
	if (gt == 3)
		hipLaunchKernelGGL(k_kq_gateup<3>, grid, dim3(KG_THREADS), 0, s, gate, up, gu_stride,
				   ids, x, h, K, E, EI, R);
	else
		hipLaunchKernelGGL(k_kq_gateup<5>, grid, dim3(KG_THREADS), 0, s, gate, up, gu_stride,
				   ids, x, h, K, E, EI, R);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_kq_down(int dt, const uint8_t *down, size_t dn_stride, const u32 *ids,
				  const float *h, float *y, int P, int E, int EI, void *stream)
{
	const dim3 grid((E + KD_ROWS - 1) / KD_ROWS, P);
	hipStream_t s = (hipStream_t)stream;
	if (dt == 3)
		hipLaunchKernelGGL(k_kq_down<3>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids, h,
				   y, E, EI);
	else
		hipLaunchKernelGGL(k_kq_down<5>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids, h,
				   y, E, EI);
	return (int)hipGetLastError();
}
