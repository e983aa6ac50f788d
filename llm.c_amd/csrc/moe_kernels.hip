/*
 * HIP kernels for the quantized MoE FFN on MI355X (gfx950, wave64).
 *
 * Stages (reference functions in parentheses):
 *   k_router        router logits, bit-exact    (matmul.c:13-33, 91-131, 169-245)
 *   k_softmax_topk  softmax + top-k (+renorm)   (nn.c:221-308, llama.c:422-427)
 *   k_gateup        gate/up dequant-GEMV + SwiGLU (nn.c:449-478, quant.c:103-155)
 *   k_down          down dequant-GEMV, K-chunk partials (nn.c:483-492)
 *   k_combine       y / (1/w) summed in slot order (olmoe.c:401-403,
 *                   tensor.c:334-353, 435-456)
 *
 * Weights stay in GGUF block layout (Q8_0: 34-byte blocks, Q4_0: 18-byte
 * blocks, quant.h:14-26).  A lane owns a "segment" of two consecutive blocks
 * (64 columns: 68 bytes Q8_0 / 36 bytes Q4_0, always 4-byte aligned because
 * rows hold an even number of blocks) and keeps the matching 64 activations in
 * registers for all the rows it visits; C lanes cover one row, 64/C rows are
 * in flight per wave step, and a row's partial sums meet in an xor-shuffle
 * tree.  The file is compiled with -ffp-contract=off: every fused
 * multiply-add is written as one.
 */
#include "moe_device.h"

/* ------------------------------------------------------------------ */
/* router: logits[t][j] = (bias[j] or 0) + dot(x[t], wr[j])            */
/* ------------------------------------------------------------------ */

/*
 * A workgroup takes RT_TOK tokens (one per wave) x 64 experts (one per lane).
 * Each thread keeps the 8 AVX2 lane accumulators of its logit: accumulator l
 * adds x[k]*w[k] for k = l, l+8, l+16, ... in increasing k with FMA
 * (dot_f32_f32, matmul.c:91-105; the tiled T>1 path of matmul.c:213-238 keeps
 * the same per-element order), then the lanes meet in the tree
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) of vector_avx2.h:126-132, and the
 * logit is fl(bias + dot) (matmul.c:24-32).
 *
 * Router rows and tokens stream through an LDS ring of RT_NST stages of
 * RT_KC columns, filled by LDS-DMA loads (global_load_lds_dwordx4, issued
 * from inline assembly so the K loop alone decides what to wait for):
 * router rows [64][RT_KC] with 16-byte chunk c of row r at slot
 * 16r + (c ^ (r & 15)) (a wave reads 64 rows conflict-free), tokens
 * [RT_TOK][RT_KC] (a wave reads its token row as a broadcast).
 */
#define RT_TOK 8
#define RT_KC 64
#define RT_NST 5
#define RT_WSZ (64 * RT_KC * 4)
#define RT_SSZ (RT_WSZ + RT_TOK * RT_KC * 4)

__device__ static inline void rt_dma16(const void *sbase, u32 voff, u32 lds)
{
	asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
		     :
		     : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds))
		     : "memory", "m0");
}

template <int N>
__device__ static inline void rt_wait_vm()
{
	static_assert(N >= 0 && N < 64, "vmcnt is six bits");
	__builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

__global__ __launch_bounds__(RT_TOK * 64) void k_router(const float *__restrict__ x,
						const float *__restrict__ wr,
						const float *__restrict__ bias,
						float *__restrict__ logits, int T, int E, int NE,
						_Float16 *__restrict__ xh)
{
	__shared__ __attribute__((aligned(16))) uint8_t ring[RT_NST * RT_SSZ];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int t0 = blockIdx.x * RT_TOK, j0 = blockIdx.y * 64;
	const int t = t0 + wave, j = j0 + lane;
	const int nc = E / RT_KC;
	const u32 l0 = (u32)(uintptr_t)(const __attribute__((address_space(3))) char *)ring;

	/* this lane's loads: RT_WQ router chunks (rows r, swizzled chunks) and,
	 * for lanes < 16, a 16-byte chunk of its wave's token row */
	constexpr int RT_WQ = 16 / RT_TOK; /* the 64 x RT_KC tile is 16 KB */
	u32 woff[RT_WQ];
#pragma unroll
	for (int q = 0; q < RT_WQ; q++) {
		const int f = (wave * RT_WQ + q) * 64 + lane, r = f >> 4, c = (f & 15) ^ (r & 15);
		woff[q] = (u32)(((size_t)(j0 + r < NE ? j0 + r : 0) * E) * 4 + 16 * c);
	}
	const u32 xoff = (u32)((size_t)(t < T ? t : 0) * E * 4 + 16 * (lane & 15));
	auto issue = [&](int s) {
		const u32 st = l0 + (u32)((s % RT_NST) * RT_SSZ);
		const float *wb = wr + (size_t)s * RT_KC, *xb = x + (size_t)s * RT_KC;
#pragma unroll
		for (int q = 0; q < RT_WQ; q++)
			rt_dma16(wb, woff[q], st + (u32)((wave * RT_WQ + q) * 1024));
		if (lane < 16)
			rt_dma16(xb, xoff, st + RT_WSZ + (u32)(wave * RT_KC * 4));
	};

	float acc[8];
#pragma unroll
	for (int l = 0; l < 8; l++)
		acc[l] = 0.0f;
#pragma unroll
	for (int s = 0; s < RT_NST - 1; s++)
		if (s < nc)
			issue(s);
	for (int s = 0; s < nc; s++) {
		if (s + RT_NST - 2 < nc)
			rt_wait_vm<(RT_NST - 2) * (RT_WQ + 1)>();
		else
			rt_wait_vm<0>();
		__syncthreads(); /* stage s landed for every wave; stage s-1 is free */
		if (s + RT_NST - 1 < nc)
			issue(s + RT_NST - 1);
		const uint8_t *st = ring + (s % RT_NST) * RT_SSZ;
		const float *xr = (const float *)(st + RT_WSZ) + wave * RT_KC;
		const uint8_t *wrow = st + lane * (RT_KC * 4);
		if (xh && blockIdx.y == 0 && t < T)
			xh[(size_t)t * E + (size_t)s * RT_KC + lane] = (_Float16)xr[lane];
#pragma unroll
		for (int k = 0; k < RT_KC; k += 8) {
			const int c = k >> 2; /* 16-byte chunks c and c+1 */
			const float4 xa = *(const float4 *)(xr + k), xb = *(const float4 *)(xr + k + 4);
			const float4 wa = *(const float4 *)(wrow + 16 * (c ^ (lane & 15)));
			const float4 wb = *(const float4 *)(wrow + 16 * ((c + 1) ^ (lane & 15)));
			acc[0] = __builtin_fmaf(xa.x, wa.x, acc[0]);
			acc[1] = __builtin_fmaf(xa.y, wa.y, acc[1]);
			acc[2] = __builtin_fmaf(xa.z, wa.z, acc[2]);
			acc[3] = __builtin_fmaf(xa.w, wa.w, acc[3]);
			acc[4] = __builtin_fmaf(xb.x, wb.x, acc[4]);
			acc[5] = __builtin_fmaf(xb.y, wb.y, acc[5]);
			acc[6] = __builtin_fmaf(xb.z, wb.z, acc[6]);
			acc[7] = __builtin_fmaf(xb.w, wb.w, acc[7]);
		}
	}
	if (t < T && j < NE) {
		const float d = ((acc[0] + acc[4]) + (acc[2] + acc[6])) +
				((acc[1] + acc[5]) + (acc[3] + acc[7]));
		logits[(size_t)t * NE + j] = (bias ? bias[j] : 0.0f) + d;
	}
}

/* ------------------------------------------------------------------ */
/* softmax + top-k, one wave per token (wave_softmax_topk)             */
/* ------------------------------------------------------------------ */

__global__ __launch_bounds__(64) void k_softmax_topk(const float *__restrict__ logits,
						     float *__restrict__ probs,
						     u32 *__restrict__ ids,
						     float *__restrict__ wout,
						     int NE, int K, int renorm)
{
	__shared__ float sp[MOE_MAX_NE];
	__shared__ u32 sid[MOE_MAX_TOPK];
	__shared__ float sw[MOE_MAX_TOPK];
	const int t = blockIdx.x;
	wave_softmax_topk(logits + (size_t)t * NE, probs ? probs + (size_t)t * NE : NULL,
			  ids + (size_t)t * K, wout + (size_t)t * K, NE, K, renorm, sp, sid, sw,
			  threadIdx.x);
}

/* ------------------------------------------------------------------ */
/* gate/up dequant-GEMV + SwiGLU                                       */
/* ------------------------------------------------------------------ */

/*
 * grid (EI / (4*rpw), P): block = 4 waves, each wave owns rpw consecutive
 * rows of gate and up for token-slot p.  C = E/64 lanes per row (a power of
 * two, 4..64), 64/C rows per wave step.
 */
template <int WT, int C>
__global__ __launch_bounds__(256) void k_gateup(const uint8_t *__restrict__ gate,
						const uint8_t *__restrict__ up,
						size_t expert_stride,
						const u32 *__restrict__ ids, int fixed_e,
						const float *__restrict__ x,
						float *__restrict__ h, int K, int E, int EI,
						int rpw)
{
	constexpr int RPS = WAVE / C;
	const int p = blockIdx.y;
	const int t = p / K;
	const int e = fixed_e >= 0 ? fixed_e : (int)ids[p];
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int seg = lane % C, sub = lane / C;
	const size_t rb = (size_t)(E / MOE_QK) * (qseg<WT>::BYTES / 2);

	const uint8_t *G = gate + (size_t)e * expert_stride + (size_t)seg * qseg<WT>::BYTES;
	const uint8_t *U = up + (size_t)e * expert_stride + (size_t)seg * qseg<WT>::BYTES;

	float xr[64];
	load_x64(x + (size_t)t * E + seg * MOE_SEG_COLS, xr);
	const float xs0 = sum32(xr), xs1 = sum32(xr + 32);

	const int row0 = (blockIdx.x * 4 + wave) * rpw;
	for (int r = 0; r < rpw; r += RPS) {
		const int row = row0 + r + sub;
		float g = qseg<WT>::dot(G + (size_t)row * rb, xr, xs0, xs1);
		float u = qseg<WT>::dot(U + (size_t)row * rb, xr, xs0, xs1);
		g = group_sum<C>(g);
		u = group_sum<C>(u);
		if (seg == 0)
			h[(size_t)p * EI + row] = (g / (1.0f + moe_expf(-g))) * u;
	}
}

/* ------------------------------------------------------------------ */
/* down dequant-GEMV over panels (K-chunk partials)                    */
/* ------------------------------------------------------------------ */

/*
 * The down matrices are stored panel by panel (panel c = block c of every
 * row, contiguous), so a thread owns one output row and walks the panels of
 * its K-chunk: a wave reads 64 consecutive blocks of a panel per load, and
 * no cross-lane sum is needed.  grid (ceil(E/256), P, kch); chunk kc covers
 * panels [kc*ppc, (kc+1)*ppc), ppc = (EI/32)/kch <= DN_MAX_PPC, whose h
 * values are staged in LDS.  Loads go out DN_BATCH panels at a time.
 */
#define DN_MAX_PPC 64
#define DN_BATCH 4
template <int WT>
__global__ __launch_bounds__(256) void k_down(const uint8_t *__restrict__ down,
					      size_t expert_stride,
					      const u32 *__restrict__ ids, int fixed_e,
					      const float *__restrict__ h,
					      float *__restrict__ ypart, int E, int EI)
{
	typedef panel_blk<WT> D;
	__shared__ __attribute__((aligned(16))) float sh[DN_MAX_PPC * MOE_QK];
	const int p = blockIdx.y, kc = blockIdx.z, kch = gridDim.z;
	const int e = fixed_e >= 0 ? fixed_e : (int)ids[p];
	const int ppc = EI / MOE_QK / kch, c0 = kc * ppc;
	const int i = blockIdx.x * 256 + threadIdx.x;
	const int ii = i < E ? i : E - 1; /* rows past E load row E-1 and store nothing */

	const float *hp = h + (size_t)p * EI + (size_t)c0 * MOE_QK;
	for (int k = threadIdx.x; k < ppc * MOE_QK; k += 256)
		sh[k] = hp[k];
	__syncthreads();

	const size_t pstride = (size_t)E * D::BB;
	const uint8_t *P0 = down + (size_t)e * expert_stride + (size_t)c0 * pstride +
			    ((D::BB * ii) & ~3);
	float y = 0.0f;
	for (int c = 0; c < ppc; c += DN_BATCH) {
		u32 d[DN_BATCH][D::DW];
#pragma unroll
		for (int u = 0; u < DN_BATCH; u++)
			if (c + u < ppc)
				load_dwords<D::DW>(P0 + (size_t)(c + u) * pstride, d[u]);
#pragma unroll
		for (int u = 0; u < DN_BATCH; u++)
			if (c + u < ppc) {
				const float *hc = sh + (c + u) * MOE_QK;
				y += D::dot(d[u], ii, hc, sum32(hc));
			}
	}
	if (i < E)
		ypart[((size_t)p * kch + kc) * E + i] = y;
}

/* K-chunks of the down GEMV for P pairs: the fewest (chunks of at most
 * DN_MAX_PPC panels) that give >= 1024 workgroups, 0 if even the fewest
 * need more than cap floats of partials */
static int down_kchunks(int E, int EI, int P, size_t cap)
{
	const int NC = EI / MOE_QK;
	int best = 0;
	for (int d = 1; d <= NC; d++) {
		if (NC % d || NC / d > DN_MAX_PPC)
			continue;
		if ((size_t)P * d * E > cap)
			break;
		best = d;
		if ((size_t)((E + 255) / 256) * P * d >= 1024)
			break;
	}
	return best;
}

/* floats of partials the down GEMV needs for any pair count up to P (the
 * chunk count falls as P grows; past 2048 pairs it is the minimum) */
extern "C" size_t moe_down_part_floats(size_t E, size_t EI, size_t P)
{
	size_t m = 0, top = P < 2048 ? P : 2048;
	for (size_t q = 1; q <= top; q++) {
		size_t v = q * (size_t)down_kchunks((int)E, (int)EI, (int)q, (size_t)-1) * E;
		m = v > m ? v : m;
	}
	size_t v = P * (size_t)down_kchunks((int)E, (int)EI, (int)P, (size_t)-1) * E;
	return v > m ? v : m;
}

/* ------------------------------------------------------------------ */
/* combine                                                             */
/* ------------------------------------------------------------------ */

__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ ypart,
						 const float *__restrict__ w,
						 float *__restrict__ out, int K, int E,
						 int kchunks)
{
	const int t = blockIdx.y;
	const int i = blockIdx.x * 256 + threadIdx.x;
	if (i >= E)
		return;
	float acc = 0.0f;
	for (int s = 0; s < K; s++) {
		const size_t p = (size_t)t * K + s;
		float y = ypart[p * kchunks * E + i];
		for (int kc = 1; kc < kchunks; kc++)
			y += ypart[(p * kchunks + kc) * E + i];
		float inv = 1.0f / (w ? w[p] : 1.0f);
		acc = acc + y / inv;
	}
	out[(size_t)t * E + i] = acc;
}

__global__ __launch_bounds__(256) void k_expf(const float *__restrict__ in,
					      float *__restrict__ out, size_t n)
{
	size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
	if (i < n)
		out[i] = moe_expf(in[i]);
}

/* plain streaming copy of n 16-byte words (calibrates the HBM byte counters) */
__global__ __launch_bounds__(256) void k_copy(const uint4 *__restrict__ src,
					      uint4 *__restrict__ dst, size_t n)
{
	for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
	     i += (size_t)gridDim.x * 256)
		dst[i] = src[i];
}

/* ------------------------------------------------------------------ */
/* launchers                                                           */
/* ------------------------------------------------------------------ */

extern "C" int moe_lanes_per_row(size_t K)
{
	size_t nseg = K / MOE_SEG_COLS;
	int c = 64;
	while (c > 1 && nseg % (size_t)c)
		c >>= 1;
	return c;
}

extern "C" int moe_kchunks(size_t K)
{
	return (int)(K / MOE_SEG_COLS / (size_t)moe_lanes_per_row(K));
}

extern "C" int moe_launch_router(const float *x, const float *wr, const float *bias,
				 float *logits, int T, int E, int NE, void *xh, void *stream)
{
	if (E % RT_KC || (size_t)NE * E * 4 > 0xffffffffull || (size_t)T * E * 4 > 0xffffffffull)
		return (int)hipErrorInvalidValue;
	dim3 grid((T + RT_TOK - 1) / RT_TOK, (NE + 63) / 64);
	hipLaunchKernelGGL(k_router, grid, dim3(RT_TOK * 64), 0, (hipStream_t)stream, x, wr,
			   bias, logits, T, E, NE, (_Float16 *)xh);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_softmax_topk(const float *logits, float *probs, uint32_t *ids,
				       float *w, int T, int NE, int K, int renorm,
				       void *stream)
{
	hipLaunchKernelGGL(k_softmax_topk, dim3(T), dim3(64), 0, (hipStream_t)stream,
			   logits, probs, ids, w, NE, K, renorm);
	return (int)hipGetLastError();
}

/* rows per wave: at least one full wave step; more rows per wave when many
 * token-slots already fill the device. */
static int pick_rpw(int rps, int P, int rows)
{
	int rpw = P >= 64 ? 16 : 4;
	if (rpw < rps)
		rpw = rps;
	while (rpw > rps && rows % (4 * rpw))
		rpw >>= 1;
	return rpw;
}

template <int WT>
static int launch_gateup_t(int C, dim3 grid, hipStream_t s, const uint8_t *gate,
			   const uint8_t *up, size_t es, const u32 *ids, int fe,
			   const float *x, float *h, int K, int E, int EI, int rpw)
{
#define GU(CC)                                                                      \
	case CC:                                                                    \
		hipLaunchKernelGGL((k_gateup<WT, CC>), grid, dim3(256), 0, s, gate, \
				   up, es, ids, fe, x, h, K, E, EI, rpw);           \
		break;
	switch (C) {
		GU(4) GU(8) GU(16) GU(32) GU(64)
	default:
		return (int)hipErrorInvalidValue;
	}
#undef GU
	return (int)hipGetLastError();
}

extern "C" int moe_launch_gateup(int wtype, const uint8_t *gate, const uint8_t *up,
				 size_t expert_stride, const uint32_t *ids, int fixed_e,
				 const float *x, float *h, int P, int K, int E, int EI,
				 void *stream)
{
	int C = moe_lanes_per_row((size_t)E);
	if (moe_kchunks((size_t)E) != 1 || C < 4)
		return (int)hipErrorInvalidValue;
	int rpw = pick_rpw(WAVE / C, P, EI);
	if (EI % (4 * rpw))
		return (int)hipErrorInvalidValue;
	dim3 grid(EI / (4 * rpw), P);
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		return launch_gateup_t<1>(C, grid, s, gate, up, expert_stride, ids, fixed_e,
					  x, h, K, E, EI, rpw);
	if (wtype == 2)
		return launch_gateup_t<2>(C, grid, s, gate, up, expert_stride, ids, fixed_e,
					  x, h, K, E, EI, rpw);
	return (int)hipErrorInvalidValue;
}

extern "C" int moe_launch_down(int wtype, const uint8_t *down, size_t expert_stride,
			       const uint32_t *ids, int fixed_e, const float *h,
			       float *ypart, size_t ypart_cap, int P, int E, int EI, int *kchunks,
			       void *stream)
{
	if (EI % MOE_QK || E % 2 || E < 2)
		return (int)hipErrorInvalidValue;
	const int kch = down_kchunks(E, EI, P, ypart_cap);
	if (kch < 1)
		return (int)hipErrorInvalidValue;
	*kchunks = kch;
	dim3 grid((E + 255) / 256, P, kch);
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		hipLaunchKernelGGL(k_down<1>, grid, dim3(256), 0, s, down, expert_stride, ids,
				   fixed_e, h, ypart, E, EI);
	else if (wtype == 2)
		hipLaunchKernelGGL(k_down<2>, grid, dim3(256), 0, s, down, expert_stride, ids,
				   fixed_e, h, ypart, E, EI);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int moe_launch_combine(const float *ypart, const float *w, float *out, int T,
				  int K, int E, int kchunks, void *stream)
{
	dim3 grid((E + 255) / 256, T);
	hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, (hipStream_t)stream, ypart, w,
			   out, K, E, kchunks);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_expf(const float *in, float *out, size_t n, void *stream)
{
	if (n == 0)
		return 0;
	dim3 grid((unsigned)((n + 255) / 256));
	hipLaunchKernelGGL(k_expf, grid, dim3(256), 0, (hipStream_t)stream, in, out, n);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_copy(const void *src, void *dst, size_t bytes, void *stream)
{
	if (bytes == 0 || bytes % 16)
		return (int)hipErrorInvalidValue;
	size_t n = bytes / 16, blocks = (n + 255) / 256;
	dim3 grid((unsigned)(blocks < 8192 ? blocks : 8192));
	hipLaunchKernelGGL(k_copy, grid, dim3(256), 0, (hipStream_t)stream, (const uint4 *)src,
			   (uint4 *)dst, n);
	return (int)hipGetLastError();
}
