/*
 * Single-precision exp that returns the same bits as glibc's expf on x86-64.
 *
 * The reference's softmax and SwiGLU call glibc's scalar expf
 * (vector_avx2.h:50-63, nn.c:247 and nn.c:477).  Routing weights must match
 * bit for bit, so the device evaluates the same published algorithm: the
 * ARM optimized-routines expf that glibc >= 2.27 ships
 * (sysdeps/ieee754/flt-32/e_expf.c).  It works in double precision:
 *
 *   x*32/ln2 = k + r, |r| <= 1/2, k integer (round to nearest via a 1.5*2^52
 *   shift);  exp(x) = 2^(k/32) * 2^(r/32),  2^(k/32) = table[k % 32] with the
 *   exponent k/32 added to its bits, and 2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3.
 *
 * On x86-64 glibc dispatches to a copy of that file built with -mfma, where
 * gcc fuses `InvLn2N * xd` into both of its uses (`z + SHIFT`, `z - kd`) and
 * every `a * b + c` of the polynomial.  The fusions are written out below with
 * fma(); the result is pinned by an exhaustive comparison against the host's
 * glibc over every float in [-104, 0] plus a stride over all of them.
 *
 * The table is 2^(i/32) rounded to double minus (i << 47); it is derived from
 * 60-digit arithmetic by gen_exp2_table.py in this directory.
 */
#ifndef MOE_EXPF_H
#define MOE_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define MOE_EXPF_FN __host__ __device__ static inline
#define MOE_EXPF_TABLE __constant__ static const
#else
#include <math.h>
#include <string.h>
#define MOE_EXPF_FN static inline
#define MOE_EXPF_TABLE static const
#endif

MOE_EXPF_TABLE uint64_t moe_exp2_tab[32] = {
	0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
	0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
	0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
	0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
	0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
	0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
	0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
	0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

MOE_EXPF_FN uint32_t moe_f2u(float f)
{
	uint32_t u;
	__builtin_memcpy(&u, &f, 4);
	return u;
}

MOE_EXPF_FN double moe_u2d(uint64_t u)
{
	double d;
	__builtin_memcpy(&d, &u, 8);
	return d;
}

MOE_EXPF_FN uint64_t moe_d2u(double d)
{
	uint64_t u;
	__builtin_memcpy(&u, &d, 8);
	return u;
}

/* the same with the 2^(i/32) table at tab (e.g. an LDS copy on the device) */
MOE_EXPF_FN float moe_expf_tab(float x, const uint64_t *tab)
{
	const double inv_ln2_n = 0x1.71547652b82fep+0 * 32; /* 32/ln2 */
	const double shift = 0x1.8p+52;
	const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
	const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
	const double c2 = 0x1.62e42ff0c52d6p-1 / 32;

	uint32_t ix = moe_f2u(x);
	uint32_t abstop = (ix >> 20) & 0x7ff;
	if (abstop >= 0x42b) {          /* |x| >= 88 or nan */
		if (ix == 0xff800000u)      /* -inf */
			return 0.0f;
		if (abstop >= 0x7f8)        /* inf or nan */
			return x + x;
		if (x > 0x1.62e42ep6f)      /* overflow */
			return __builtin_inff();
		if (x < -0x1.9fe368p6f)     /* underflow to zero */
			return 0.0f;
	}
	double xd = (double)x;
	double kd = __builtin_fma(inv_ln2_n, xd, shift);
	uint64_t ki = moe_d2u(kd);
	kd -= shift;
	double r = __builtin_fma(inv_ln2_n, xd, -kd);
	uint64_t t = tab[ki % 32];
	t += ki << 47;
	double s = moe_u2d(t);
	double z = __builtin_fma(c0, r, c1);
	double r2 = r * r;
	double y = __builtin_fma(c2, r, 1.0);
	y = __builtin_fma(z, r2, y);
	y = y * s;
	return (float)y;
}

MOE_EXPF_FN float moe_expf(float x)
{
	return moe_expf_tab(x, moe_exp2_tab);
}

#endif
