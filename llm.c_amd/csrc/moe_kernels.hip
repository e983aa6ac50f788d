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
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_expf.h"
#include "moe_internal.h"

typedef uint32_t u32;

#define WAVE 64

/* ------------------------------------------------------------------ */
/* helpers                                                            */
/* ------------------------------------------------------------------ */

__device__ static inline float f16_bits_to_f32(u32 h)
{
	return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

/* 16 bytes read from a 4-byte aligned address (one global_load_dwordx4). */
struct __attribute__((packed, aligned(4))) dw4 {
	u32 v[4];
};

template <int N>
__device__ static inline void load_dwords(const uint8_t *p, u32 (&d)[N])
{
	const dw4 *q = (const dw4 *)p;
#pragma unroll
	for (int i = 0; i < N / 4; i++) {
		dw4 t = q[i];
		d[4 * i + 0] = t.v[0];
		d[4 * i + 1] = t.v[1];
		d[4 * i + 2] = t.v[2];
		d[4 * i + 3] = t.v[3];
	}
#pragma unroll
	for (int i = (N / 4) * 4; i < N; i++)
		d[i] = ((const u32 *)p)[i];
}

/* Q8_0 segment: 17 dwords.  Block 0 = bytes 0..33 (scale in bytes 0-1,
 * quants 2..33, i.e. misaligned by 2), block 1 = bytes 34..67 (scale 34-35,
 * quants 36..67 = dwords 9..16). */
__device__ static inline float seg_dot_q8_0(const u32 (&d)[17], const float (&x)[64])
{
	float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
	for (int k = 0; k < 8; k++) {
		u32 q = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
#pragma unroll
		for (int b = 0; b < 4; b++)
			s0 = __builtin_fmaf((float)(int)(int8_t)(q >> (8 * b)), x[4 * k + b], s0);
	}
#pragma unroll
	for (int k = 0; k < 8; k++) {
		u32 q = d[9 + k];
#pragma unroll
		for (int b = 0; b < 4; b++)
			s1 = __builtin_fmaf((float)(int)(int8_t)(q >> (8 * b)), x[32 + 4 * k + b], s1);
	}
	float d0 = f16_bits_to_f32(d[0]);
	float d1 = f16_bits_to_f32(d[8] >> 16);
	return __builtin_fmaf(d1, s1, d0 * s0);
}

/* Q4_0 segment: 9 dwords.  Block 0 = bytes 0..17 (scale 0-1, packed nibbles
 * 2..17), block 1 = bytes 18..35 (scale 18-19, nibbles 20..35 = dwords 5..8).
 * Byte j of a block holds element j (low nibble) and j+16 (high nibble),
 * each biased by 8 (quant.c:126-155). */
__device__ static inline float seg_dot_q4_0(const u32 (&d)[9], const float (&x)[64])
{
	float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		u32 q = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
#pragma unroll
		for (int b = 0; b < 4; b++) {
			int lo = (int)((q >> (8 * b)) & 15u) - 8;
			int hi = (int)((q >> (8 * b + 4)) & 15u) - 8;
			s0 = __builtin_fmaf((float)lo, x[4 * k + b], s0);
			s0 = __builtin_fmaf((float)hi, x[16 + 4 * k + b], s0);
		}
	}
#pragma unroll
	for (int k = 0; k < 4; k++) {
		u32 q = d[5 + k];
#pragma unroll
		for (int b = 0; b < 4; b++) {
			int lo = (int)((q >> (8 * b)) & 15u) - 8;
			int hi = (int)((q >> (8 * b + 4)) & 15u) - 8;
			s1 = __builtin_fmaf((float)lo, x[32 + 4 * k + b], s1);
			s1 = __builtin_fmaf((float)hi, x[48 + 4 * k + b], s1);
		}
	}
	float d0 = f16_bits_to_f32(d[0]);
	float d1 = f16_bits_to_f32(d[4] >> 16);
	return __builtin_fmaf(d1, s1, d0 * s0);
}

template <int WT> struct qseg;
template <> struct qseg<1> {
	static constexpr int BYTES = 68;
	static constexpr int DW = 17;
	__device__ static inline float dot(const uint8_t *p, const float (&x)[64])
	{
		u32 d[17];
		load_dwords<17>(p, d);
		return seg_dot_q8_0(d, x);
	}
};
template <> struct qseg<2> {
	static constexpr int BYTES = 36;
	static constexpr int DW = 9;
	__device__ static inline float dot(const uint8_t *p, const float (&x)[64])
	{
		u32 d[9];
		load_dwords<9>(p, d);
		return seg_dot_q4_0(d, x);
	}
};

/* sum over the C consecutive lanes of a row group (C a power of two) */
template <int C>
__device__ static inline float group_sum(float v)
{
#pragma unroll
	for (int off = C / 2; off >= 1; off >>= 1)
		v += __shfl_xor(v, off, WAVE);
	return v;
}

__device__ static inline void load_x64(const float *src, float (&x)[64])
{
	const float4 *s4 = (const float4 *)src;
#pragma unroll
	for (int i = 0; i < 16; i++) {
		float4 v = s4[i];
		x[4 * i + 0] = v.x;
		x[4 * i + 1] = v.y;
		x[4 * i + 2] = v.z;
		x[4 * i + 3] = v.w;
	}
}

/* ------------------------------------------------------------------ */
/* router: logits[t][j] = (bias[j] or 0) + dot(x[t], wr[j])            */
/* ------------------------------------------------------------------ */

/* Eight threads per logit; thread l accumulates elements l, l+8, ... with
 * FMA in increasing order (one AVX2 lane), then the lanes meet in the tree
 * ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) of vector_avx2.h:126-132. */
__global__ __launch_bounds__(64) void k_router(const float *__restrict__ x,
					       const float *__restrict__ wr,
					       const float *__restrict__ bias,
					       float *__restrict__ logits, int E, int NE)
{
	int t = blockIdx.y;
	int j = blockIdx.x * 8 + (threadIdx.x >> 3);
	int l = threadIdx.x & 7;
	float acc = 0.0f;
	if (j < NE) {
		const float *xr = x + (size_t)t * E;
		const float *w = wr + (size_t)j * E;
		for (int i = l; i < E; i += 8)
			acc = __builtin_fmaf(xr[i], w[i], acc);
	}
	acc = acc + __shfl_xor(acc, 4, 8);
	acc = acc + __shfl_xor(acc, 2, 8);
	acc = acc + __shfl_xor(acc, 1, 8);
	if (j < NE && l == 0)
		logits[(size_t)t * NE + j] = (bias ? bias[j] : 0.0f) + acc;
}

/* ------------------------------------------------------------------ */
/* softmax + top-k, one wave per token                                 */
/* ------------------------------------------------------------------ */

/*
 * softmax_1d (nn.c:221-262): e_i = expf(v_i - max); lane sums s_l over the
 * 8-wide chunks in order, the reduction tree, then the scalar tail; p = e/sum.
 *
 * top_k (nn.c:276-308) seeds all k slots with element 0 and inserts later
 * elements only when strictly greater than the current minimum.  Its result
 * in closed form: rank_i = #{j : p_j > p_i or (p_j == p_i and j < i)};
 * r0 = rank of element 0.  Element i != 0 lands in slot k-1-rank_i iff
 * rank_i < min(r0, k); when r0 < k, slots 0..k-1-r0 hold copies of element 0.
 * Slots ascend by weight, later indices below earlier ones among ties.
 */
__global__ __launch_bounds__(64) void k_softmax_topk(const float *__restrict__ logits,
						     float *__restrict__ probs,
						     u32 *__restrict__ ids,
						     float *__restrict__ wout,
						     int NE, int K, int renorm)
{
	__shared__ float sp[MOE_MAX_NE];
	__shared__ u32 sid[MOE_MAX_TOPK];
	__shared__ float sw[MOE_MAX_TOPK];
	__shared__ int srank0;
	__shared__ float ssum;

	const int t = blockIdx.x, lane = threadIdx.x;
	const float *row = logits + (size_t)t * NE;

	float mx = -__builtin_inff();
	for (int i = lane; i < NE; i += WAVE)
		mx = fmaxf(mx, row[i]);
#pragma unroll
	for (int off = 32; off >= 1; off >>= 1)
		mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));

	for (int i = lane; i < NE; i += WAVE)
		sp[i] = moe_expf(row[i] - mx);
	__syncthreads();

	const int nv = NE - NE % 8;
	float s = 0.0f;
	if (lane < 8)
		for (int c = 0; c < nv; c += 8)
			s = s + sp[c + lane];
	s = s + __shfl_xor(s, 4, 8);
	s = s + __shfl_xor(s, 2, 8);
	s = s + __shfl_xor(s, 1, 8);
	if (lane == 0) {
		for (int i = nv; i < NE; i++)
			s += sp[i];
		ssum = s;
	}
	__syncthreads();
	const float sum = ssum;
	for (int i = lane; i < NE; i += WAVE) {
		float p = sp[i] / sum;
		sp[i] = p;
		if (probs)
			probs[(size_t)t * NE + i] = p;
	}
	__syncthreads();

	int myrank[MOE_MAX_NE / WAVE];
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
		int i = lane + r * WAVE;
		int rank = 0;
		if (i < NE) {
			float pi = sp[i];
			for (int j = 0; j < NE; j++) {
				float pj = sp[j];
				rank += (pj > pi) || (pj == pi && j < i);
			}
			if (i == 0)
				srank0 = rank;
		}
		myrank[r] = rank;
	}
	__syncthreads();
	const int r0 = srank0;
	const int lim = r0 < K ? r0 : K;
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
		int i = lane + r * WAVE;
		if (i > 0 && i < NE && myrank[r] < lim) {
			sid[K - 1 - myrank[r]] = (u32)i;
			sw[K - 1 - myrank[r]] = sp[i];
		}
	}
	if (r0 < K)
		for (int slot = lane; slot < K - r0; slot += WAVE) {
			sid[slot] = 0;
			sw[slot] = sp[0];
		}
	__syncthreads();
	if (lane == 0) {
		if (renorm) {
			float ws = 0.0f;
			for (int e = 0; e < K; e++)
				ws += sw[e];
			for (int e = 0; e < K; e++)
				sw[e] /= ws;
		}
		for (int e = 0; e < K; e++) {
			ids[(size_t)t * K + e] = sid[e];
			wout[(size_t)t * K + e] = sw[e];
		}
	}
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

	const int row0 = (blockIdx.x * 4 + wave) * rpw;
	for (int r = 0; r < rpw; r += RPS) {
		const int row = row0 + r + sub;
		float g = qseg<WT>::dot(G + (size_t)row * rb, xr);
		float u = qseg<WT>::dot(U + (size_t)row * rb, xr);
		g = group_sum<C>(g);
		u = group_sum<C>(u);
		if (seg == 0)
			h[(size_t)p * EI + row] = (g / (1.0f + moe_expf(-g))) * u;
	}
}

/* ------------------------------------------------------------------ */
/* down dequant-GEMV (K-chunk partials)                                */
/* ------------------------------------------------------------------ */

/* grid (E / (4*rpw), P, kchunks); C lanes per row over chunk kc's
 * C segments (C*64 columns). */
template <int WT, int C>
__global__ __launch_bounds__(256) void k_down(const uint8_t *__restrict__ down,
					      size_t expert_stride,
					      const u32 *__restrict__ ids, int fixed_e,
					      const float *__restrict__ h,
					      float *__restrict__ ypart, int E, int EI,
					      int rpw)
{
	constexpr int RPS = WAVE / C;
	const int p = blockIdx.y, kc = blockIdx.z, kch = gridDim.z;
	const int e = fixed_e >= 0 ? fixed_e : (int)ids[p];
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int seg = kc * C + lane % C, sub = lane / C;
	const size_t rb = (size_t)(EI / MOE_QK) * (qseg<WT>::BYTES / 2);

	const uint8_t *D = down + (size_t)e * expert_stride + (size_t)seg * qseg<WT>::BYTES;

	float xr[64];
	load_x64(h + (size_t)p * EI + seg * MOE_SEG_COLS, xr);

	const int row0 = (blockIdx.x * 4 + wave) * rpw;
	for (int r = 0; r < rpw; r += RPS) {
		const int row = row0 + r + sub;
		float y = group_sum<C>(qseg<WT>::dot(D + (size_t)row * rb, xr));
		if (lane % C == 0)
			ypart[((size_t)p * kch + kc) * E + row] = y;
	}
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
				 float *logits, int T, int E, int NE, void *stream)
{
	dim3 grid((NE + 7) / 8, T);
	hipLaunchKernelGGL(k_router, grid, dim3(64), 0, (hipStream_t)stream, x, wr,
			   bias, logits, E, NE);
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

template <int WT>
static int launch_down_t(int C, dim3 grid, hipStream_t s, const uint8_t *down,
			 size_t es, const u32 *ids, int fe, const float *h, float *yp,
			 int E, int EI, int rpw)
{
#define DN(CC)                                                                      \
	case CC:                                                                    \
		hipLaunchKernelGGL((k_down<WT, CC>), grid, dim3(256), 0, s, down, es, \
				   ids, fe, h, yp, E, EI, rpw);                    \
		break;
	switch (C) {
		DN(4) DN(8) DN(16) DN(32) DN(64)
	default:
		return (int)hipErrorInvalidValue;
	}
#undef DN
	return (int)hipGetLastError();
}

extern "C" int moe_launch_down(int wtype, const uint8_t *down, size_t expert_stride,
			       const uint32_t *ids, int fixed_e, const float *h,
			       float *ypart, int P, int K, int E, int EI, void *stream)
{
	(void)K;
	int C = moe_lanes_per_row((size_t)EI);
	if (C < 4)
		return (int)hipErrorInvalidValue;
	int kch = moe_kchunks((size_t)EI);
	int rpw = pick_rpw(WAVE / C, P * kch, E);
	if (E % (4 * rpw))
		return (int)hipErrorInvalidValue;
	dim3 grid(E / (4 * rpw), P, kch);
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		return launch_down_t<1>(C, grid, s, down, expert_stride, ids, fixed_e, h,
					ypart, E, EI, rpw);
	if (wtype == 2)
		return launch_down_t<2>(C, grid, s, down, expert_stride, ids, fixed_e, h,
					ypart, E, EI, rpw);
	return (int)hipErrorInvalidValue;
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
