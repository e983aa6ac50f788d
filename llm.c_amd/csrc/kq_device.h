/*
 * kq_device.h - device arithmetic of the K-quant expert products, shared by
 * kq_moe.hip (the per-pair kernels) and moe_decode.hip (the decode-sized
 * layer): the Q8_K quantizer of one 256-value block (quantize_row_q8,
 * quant.c:627-654), the integer sums of a Q4_K / Q6_K super-block against
 * a staged Q8_K block (the pieces of dot_q4_K_q8_K / dot_q6_K_q8_K,
 * quant_avx2.h:8-209), and accumulator l's part of the fp32 K-quant dot of a
 * staged down super-block (dot_f32_q4_K / dot_f32_q6_K, quant.c:198-418).
 */
#pragma once
#include "moe_device.h"

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
/* down dots                                                            */
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
				/* (q - 32) * vs as fma(q, vs, -32 vs): the exact product
				 * rounded once, as the reference's (float)(q - 32) * vs
				 * (-32 vs is exact), one instruction fewer */
				const float vs = d * (float)sc[8 * c + 2 * g + hf];
				const float nvs = -32.0f * vs;
#pragma unroll
				for (int m = 0; m < 2; m++) {
					const int lo = (int)ql[c][hf][m][g & 1];
					const int q = (g < 2 ? lo & 0xF : lo >> 4) |
						      (((int)(qh[c][hf][m] >> (2 * g)) & 3) << 4);
					const float vt = fmaf((float)q, vs, nvs);
					acc = fmaf(vt, hv[16 * c + 4 * g + 2 * hf + m], acc);
				}
			}
}

