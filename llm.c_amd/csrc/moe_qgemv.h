/*
 * moe_qgemv.h - the row-group loop of the dense quantized product
 * (moe_qgemv.hip), shared with the model kernels (lm_kernels.hip), which
 * stage their token themselves (a normalised residual stream) and watch
 * the outputs (the greedy pick of the lm_head).
 */
#ifndef MOE_QGEMV_H
#define MOE_QGEMV_H

#include "moe_device.h"
#include "moe_internal.h"

#define QG_WAVES 4
#define QG_LDS_MAX 65536 /* bytes of staged tokens: QG_LDS_MAX / (K/64 * 68 * 4) at a time */
#define QG_GRID 768      /* workgroups when the caller passes no grid */

#define QG_ARGS                                                                         \
	const uint8_t *__restrict__ W, size_t rb, int N, int K, const float *__restrict__ x, \
		int T, int tgmax, const float *__restrict__ add, int add_rows,             \
		float *__restrict__ out

/* no watcher of the outputs */
struct QgNoHook {
	__device__ void operator()(int, float) const {}
};

/*
 * ONE: T == 1.  STAGED: the caller has put the one token in LDS (segment
 * layout, SEG_STRIDE floats per 64 columns) and synchronised.  hook(row,
 * value) sees every stored output of a one-token call (lanes with seg == 0).
 */
template <int WT, int C, bool ONE, bool STAGED = false, class Hook = QgNoHook>
__device__ __forceinline__ static void qgemv_body(float *sx, QG_ARGS, Hook hook = Hook())
{
	constexpr int RPS = WAVE / C; /* rows per wave and group */
	constexpr int DW = qseg<WT>::DW;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int seg = lane % C, sub = lane / C;
	const int nseg = K / MOE_SEG_COLS; /* == C */
	const int tstride = nseg * SEG_STRIDE;
	const int ngroups = (N + QG_WAVES * RPS - 1) / (QG_WAVES * RPS);
	const bool once = T <= tgmax; /* every token fits in LDS: stage them once */

	auto stage = [&](int t0, int tg) {
		for (int i = threadIdx.x; i < tg * K / 4; i += QG_WAVES * WAVE) {
			const int t = i / (K / 4), c4 = i % (K / 4); /* float4 c4 of token t */
			const float4 v = ((const float4 *)(x + (size_t)(t0 + t) * K))[c4];
			*(float4 *)(sx + t * tstride + (c4 / 16) * SEG_STRIDE + 4 * (c4 % 16)) = v;
		}
	};
	/* rows past N repeat the last row (their results are not stored) */
	auto load = [&](int g, u32(&d)[DW]) {
		const int row = min(g * (QG_WAVES * RPS) + wave * RPS + sub, N - 1);
		load_dwords<DW>(W + (size_t)row * rb + (size_t)seg * qseg<WT>::BYTES, d);
	};
	auto dot = [&](const u32(&d)[DW], const float(&xr)[64], float xs0, float xs1) {
		float v;
		if constexpr (WT == 1)
			v = seg_dot_q8_0(d, xr, xs0, xs1);
		else
			v = seg_dot_q4_0(d, xr, xs0, xs1);
		return group_sum<C>(v);
	};
	auto store = [&](int g, int t, float v) {
		const int row = g * (QG_WAVES * RPS) + wave * RPS + sub;
		if (seg == 0 && row < N) {
			const size_t o = (size_t)t * N + row;
			const float r = (add ? add[add_rows ? o : (size_t)row] : 0.0f) + v;
			out[o] = r;
			if constexpr (ONE)
				hook(row, r);
		}
	};

	int g = blockIdx.x;
	if (g >= ngroups)
		return; /* the whole workgroup: no barrier below is left waiting */
	u32 dn[DW];
	load(g, dn);
	if constexpr (!ONE) {
		if (!once) {
			/* more tokens than LDS holds: token groups outside, this
			 * workgroup's row groups inside, so each token group is
			 * staged once (a row group's weights load again per token
			 * group, mostly from L2); the same dots as below */
			for (int t0 = 0; t0 < T; t0 += tgmax) {
				const int tg = min(tgmax, T - t0);
				__syncthreads(); /* the previous token group's readers are done */
				stage(t0, tg);
				__syncthreads();
				if (t0 > 0)
					load(blockIdx.x, dn);
				for (int gg = blockIdx.x; gg < ngroups; gg += gridDim.x) {
					u32 d[DW];
#pragma unroll
					for (int i = 0; i < DW; i++)
						d[i] = dn[i];
					if (gg + (int)gridDim.x < ngroups)
						load(gg + gridDim.x, dn);
					for (int t = 0; t < tg; t++) {
						float xr[64];
						lds_x64(sx + t * tstride, seg, xr);
						store(gg, t0 + t, dot(d, xr, sum32(xr), sum32(xr + 32)));
					}
				}
			}
			return;
		}
	}
	if (!STAGED && once) {
		stage(0, T);
		__syncthreads();
	}
	float x1s0 = 0.0f, x1s1 = 0.0f; /* the one token's block sums; its columns stay in LDS */
	const float(&x1)[64] = *(const float(*)[64])(sx + seg * SEG_STRIDE);
	if constexpr (ONE) {
		float xr[64];
		lds_x64(sx, seg, xr);
		x1s0 = sum32(xr);
		x1s1 = sum32(xr + 32);
	}
	/* groups blockIdx.x, + gridDim.x, ...: the next group's weights load
	 * while this one's dots run */
	for (; g < ngroups; g += gridDim.x) {
		u32 d[DW];
#pragma unroll
		for (int i = 0; i < DW; i++)
			d[i] = dn[i];
		if (g + (int)gridDim.x < ngroups)
			load(g + gridDim.x, dn);
		if constexpr (ONE) {
			store(g, 0, dot(d, x1, x1s0, x1s1));
			continue;
		}
		for (int t = 0; t < T; t++) { /* every token is staged */
			float xr[64];
			lds_x64(sx + t * tstride, seg, xr);
			store(g, t, dot(d, xr, sum32(xr), sum32(xr + 32)));
		}
	}
}

#endif
