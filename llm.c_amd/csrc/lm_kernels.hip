/*
 * Kernels of the whole-model decode step around the MoE layer (hip_lm.c):
 *
 *   k_embed          token row of token_embd, dequantized (tensor_pick_rows,
 *                    tensor.c:263-294), the token taken from the prompt or
 *                    from the previous step's greedy pick
 *   k_add_rmsnorm    h = a (+ b), x = rms_norm(h) * w (nn.c:8-51 with the
 *                    residual tensor_add, tensor.c:334-353, in front)
 *   k_qk_rope_kv     full-vector RMSNorm of q and k (OLMoE's attn_q_norm /
 *                    attn_k_norm, olmoe.c:454-458), RoPE on consecutive pairs
 *                    (rope_apply, nn.c:192-219), k and v into the cache row
 *   k_attn_part      one (head, chunk of positions): scores q.k / sqrt(HLEN),
 *                    the chunk's max, sum of exp and exp-weighted sum of v
 *   k_attn_merge     the chunks of a head merged into softmax(scores) . V
 *                    (olmoe.c:302-320; the flash-decoding split of it)
 *   k_argmax         the greedy pick over the logits (main.c:189-193: the
 *                    first maximum wins), and the step's counters advanced
 *   k_kv_rotate      kvcache_rotate (kvcache.c:31-56): keep the last entries
 *
 * Every kernel reads the step's token, position and cache row from a small
 * device state block (LmState), so one captured HIP graph serves every step.
 * Compiled with -ffp-contract=off: fused multiply-adds only where written.
 */
#include "moe_device.h"
#include "lm_internal.h"

#define LM_NT 256 /* threads of the single-workgroup kernels */

/* sum over the workgroup of one float per thread (LM_NT threads) */
__device__ static inline float block_sum(float v, float *red)
{
	for (int o = WAVE / 2; o > 0; o >>= 1)
		v += __shfl_xor(v, o, WAVE);
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	__syncthreads();
	if (lane == 0)
		red[wave] = v;
	__syncthreads();
	float s = 0.0f;
#pragma unroll
	for (int w = 0; w < LM_NT / WAVE; w++)
		s += red[w];
	return s;
}

__device__ static inline float block_max(float v, float *red)
{
	for (int o = WAVE / 2; o > 0; o >>= 1)
		v = fmaxf(v, __shfl_xor(v, o, WAVE));
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	__syncthreads();
	if (lane == 0)
		red[wave] = v;
	__syncthreads();
	float m = red[0];
#pragma unroll
	for (int w = 1; w < LM_NT / WAVE; w++)
		m = fmaxf(m, red[w]);
	return m;
}

/* ---------------------------------------------------------------------- */

/* the step's token: the prompt's while it lasts, then the last pick */
__device__ static inline int step_token(const LmState *st, const int *prompt)
{
	return st->step < st->n_prompt ? prompt[st->step] : st->tok;
}

/* hidden[E] = dequantized row tok of token_embd (quant.c:157-196: d * q) */
template <int WT>
__global__ __launch_bounds__(LM_NT) void k_embed(const uint8_t *__restrict__ wte, int E,
						 const LmState *__restrict__ st,
						 const int *__restrict__ prompt, float *__restrict__ hidden)
{
	const int tok = step_token(st, prompt);
	constexpr int BB = WT == 1 ? 34 : 18;
	const uint8_t *row = wte + (size_t)tok * (size_t)(E / 32) * BB;
	for (int i = threadIdx.x; i < E; i += LM_NT) {
		const uint8_t *b = row + (size_t)(i / 32) * BB;
		const float d = f16_bits_to_f32((u32)b[0] | ((u32)b[1] << 8));
		const int j = i % 32;
		float q;
		if (WT == 1)
			q = (float)(int8_t)b[2 + j];
		else
			q = (float)((j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4)) - 8);
		hidden[i] = d * q;
	}
}

/*
 * h = a + b (b may be NULL: h = a, not written back), x = (h / rms) * w,
 * rms = sqrtf(sum(h^2) / E + 1e-5f).  One workgroup; E <= 32 * LM_NT.
 */
__global__ __launch_bounds__(LM_NT) void k_add_rmsnorm(const float *__restrict__ a,
						       const float *__restrict__ b,
						       float *__restrict__ h,
						       const float *__restrict__ w,
						       float *__restrict__ x, int E)
{
	__shared__ float red[LM_NT / WAVE];
	float v[32];
	float s = 0.0f;
#pragma unroll
	for (int k = 0; k < 32; k++) {
		const int i = threadIdx.x + k * LM_NT;
		v[k] = 0.0f;
		if (i < E) {
			v[k] = b ? a[i] + b[i] : a[i];
			const float sq = v[k] * v[k];
			s = s + sq;
		}
	}
	const float sum = block_sum(s, red);
	const float rms = sqrtf(sum / (float)E + 1e-5f);
#pragma unroll
	for (int k = 0; k < 32; k++) {
		const int i = threadIdx.x + k * LM_NT;
		if (i < E) {
			if (b)
				h[i] = v[k];
			const float r = v[k] / rms;
			x[i] = r * w[i];
		}
	}
}

/*
 * qkv = [q (H*HL) | k (KH*HL) | v (KH*HL)].  With q_norm / k_norm: the
 * full-vector RMSNorm of q and of k first.  Then RoPE at the step's
 * position on q and k: pair (2i, 2i+1) of each head turns by pos * freq[i]
 * (freq from the host: 1 / powf(theta, 2i / HL), nn.c:205), x0' =
 * x0 cos - x1 sin, x1' = x0 sin + x1 cos (the reference's clang build
 * contracts each into one FMA, left product first).  k and v go to cache
 * row `size` of every kv head ([KH][C][HL] per layer).
 */
__global__ __launch_bounds__(LM_NT) void k_qk_rope_kv(float *__restrict__ qkv,
						      const float *__restrict__ q_norm,
						      const float *__restrict__ k_norm,
						      const float *__restrict__ freq,
						      const LmState *__restrict__ st,
						      float *__restrict__ kc, float *__restrict__ vc,
						      int H, int KH, int HL, int C)
{
	__shared__ float red[LM_NT / WAVE];
	const int EQ = H * HL, EK = KH * HL;
	float *q = qkv, *k = qkv + EQ;
	const float *v = qkv + EQ + EK;
	/* olmoe_decode: a position past the context is replaced by the cache
	 * size (olmoe.c:514-515) */
	const int pos = st->pos < C ? st->pos : st->size;
	const int row = st->size;
	if (q_norm) {
		for (int part = 0; part < 2; part++) {
			float *t = part ? k : q;
			const float *w = part ? k_norm : q_norm;
			const int n = part ? EK : EQ;
			float s = 0.0f;
			for (int i = threadIdx.x; i < n; i += LM_NT) {
				const float sq = t[i] * t[i];
				s = s + sq;
			}
			const float rms = sqrtf(block_sum(s, red) / (float)n + 1e-5f);
			for (int i = threadIdx.x; i < n; i += LM_NT) {
				const float r = t[i] / rms;
				t[i] = r * w[i];
			}
			__syncthreads();
		}
	}
	const int half = HL / 2;
	for (int p = threadIdx.x; p < (H + KH) * half; p += LM_NT) {
		const int hh = p / half, i = p % half;
		float *x = hh < H ? q + hh * HL : k + (hh - H) * HL;
		const float angle = (float)pos * freq[i];
		const float c = cosf(angle), s = sinf(angle);
		const float x0 = x[2 * i], x1 = x[2 * i + 1];
		const float y0 = __builtin_fmaf(x0, c, -(x1 * s));
		const float y1 = __builtin_fmaf(x0, s, x1 * c);
		x[2 * i] = y0;
		x[2 * i + 1] = y1;
		if (hh >= H) {
			float *kr = kc + ((size_t)(hh - H) * C + row) * HL;
			kr[2 * i] = y0;
			kr[2 * i + 1] = y1;
		}
	}
	for (int i = threadIdx.x; i < EK; i += LM_NT)
		vc[((size_t)(i / HL) * C + row) * HL + i % HL] = v[i];
}

/*
 * One (query head h, chunk c of LM_CHUNK positions) of decode attention
 * over the cache rows [lo, AT), AT = size + 1 (lo > 0 with a sliding
 * window).  Thread t: position t / 4 of the chunk, dims (t % 4) * 32 ..
 * +31 for the scores; then dim t % HL over half the chunk's positions for
 * the v sum.  Writes part[h][c] = {max m, sum l of exp(s - m), o[HL] =
 * sum exp(s - m) v}; an empty chunk writes m = -inf, l = 0.
 */
__global__ __launch_bounds__(LM_NT) void k_attn_part(const float *__restrict__ q,
						     const float *__restrict__ kc,
						     const float *__restrict__ vc,
						     const LmState *__restrict__ st,
						     float *__restrict__ part, int H, int KH, int C,
						     int window, float scale_div)
{
	constexpr int HL = LM_HLEN, CH = LM_CHUNK;
	__shared__ float sq[HL];
	__shared__ float sp[CH];
	__shared__ float red[LM_NT / WAVE];
	__shared__ float so[LM_NT];
	const int h = blockIdx.x, c = blockIdx.y, nchunk = gridDim.y;
	const int AT = st->size + 1;
	const int lo = window > 0 && AT > window ? AT - window : 0;
	const int j0 = lo + c * CH;
	float *pp = part + ((size_t)h * nchunk + c) * (HL + 2);
	if (j0 >= AT) {
		if (threadIdx.x == 0) {
			pp[0] = -INFINITY;
			pp[1] = 0.0f;
		}
		return;
	}
	const int n = min(CH, AT - j0);
	const int kh = h / (H / KH);
	const float *K = kc + ((size_t)kh * C + j0) * HL, *V = vc + ((size_t)kh * C + j0) * HL;
	if (threadIdx.x < HL)
		sq[threadIdx.x] = q[h * HL + threadIdx.x];
	__syncthreads();
	/* scores: 4 threads per position, 32 dims each */
	{
		const int j = threadIdx.x / 4, d0 = (threadIdx.x % 4) * 32;
		float acc = 0.0f;
		if (j < n) {
			const float4 *k4 = (const float4 *)(K + (size_t)j * HL + d0);
#pragma unroll
			for (int u = 0; u < 8; u++) {
				const float4 kv = k4[u];
				acc = __builtin_fmaf(sq[d0 + 4 * u + 0], kv.x, acc);
				acc = __builtin_fmaf(sq[d0 + 4 * u + 1], kv.y, acc);
				acc = __builtin_fmaf(sq[d0 + 4 * u + 2], kv.z, acc);
				acc = __builtin_fmaf(sq[d0 + 4 * u + 3], kv.w, acc);
			}
		}
		acc += __shfl_xor(acc, 1, WAVE);
		acc += __shfl_xor(acc, 2, WAVE);
		if (threadIdx.x % 4 == 0 && j < CH)
			sp[j] = j < n ? acc / scale_div : -INFINITY;
	}
	__syncthreads();
	const float m = block_max(threadIdx.x < CH ? sp[threadIdx.x] : -INFINITY, red);
	float e = 0.0f;
	if (threadIdx.x < CH) {
		e = threadIdx.x < n ? moe_expf(sp[threadIdx.x] - m) : 0.0f;
		sp[threadIdx.x] = e;
	}
	const float l = block_sum(e, red); /* its barriers also publish sp */
	/* o[d] = sum_j e_j v[j][d]: two halves of the positions */
	{
		const int d = threadIdx.x % HL, half = threadIdx.x / HL;
		float o = 0.0f;
		for (int j = half; j < n; j += LM_NT / HL)
			o = __builtin_fmaf(sp[j], V[(size_t)j * HL + d], o);
		so[threadIdx.x] = o;
	}
	__syncthreads();
	if (threadIdx.x < HL) {
		float o = so[threadIdx.x];
		for (int k = 1; k < LM_NT / HL; k++)
			o += so[threadIdx.x + k * HL];
		pp[2 + threadIdx.x] = o;
	}
	if (threadIdx.x == 0) {
		pp[0] = m;
		pp[1] = l;
	}
}

/* out[h * HL + d] = sum_c exp(m_c - M) o_c[d] / sum_c exp(m_c - M) l_c:
 * one workgroup of HL threads per head */
__global__ __launch_bounds__(LM_HLEN) void k_attn_merge(const float *__restrict__ part,
							float *__restrict__ out, int nchunk)
{
	constexpr int HL = LM_HLEN;
	const int h = blockIdx.x, d = threadIdx.x;
	const float *pp = part + (size_t)h * nchunk * (HL + 2);
	float M = -INFINITY;
	for (int c = 0; c < nchunk; c++)
		M = fmaxf(M, pp[(size_t)c * (HL + 2)]);
	float L = 0.0f, o = 0.0f;
	for (int c = 0; c < nchunk; c++) {
		const float *pc = pp + (size_t)c * (HL + 2);
		if (pc[1] == 0.0f)
			continue;
		const float f = moe_expf(pc[0] - M);
		L = __builtin_fmaf(f, pc[1], L);
		o = __builtin_fmaf(f, pc[2 + d], o);
	}
	out[h * HL + d] = o / L;
}

/*
 * The greedy pick: the first index of the maximum (main.c:189-193 keeps
 * the lowest index among equal maxima), written as the next token and into
 * tokens[step]; then the counters advance (step, pos, size).  One
 * workgroup of LM_ARG_NT threads.
 */
__global__ __launch_bounds__(LM_ARG_NT) void k_argmax(const float *__restrict__ logits, int V,
						      LmState *__restrict__ st,
						      int *__restrict__ tokens)
{
	__shared__ float sv[LM_ARG_NT / WAVE];
	__shared__ int si[LM_ARG_NT / WAVE];
	float bv = -INFINITY;
	int bi = 0x7fffffff;
	for (int i = threadIdx.x; i < V; i += LM_ARG_NT) {
		const float v = logits[i];
		if (v > bv) { /* increasing i: keeps the first of equal values */
			bv = v;
			bi = i;
		}
	}
	for (int o = WAVE / 2; o > 0; o >>= 1) {
		const float ov = __shfl_xor(bv, o, WAVE);
		const int oi = __shfl_xor(bi, o, WAVE);
		if (ov > bv || (ov == bv && oi < bi)) {
			bv = ov;
			bi = oi;
		}
	}
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	if (lane == 0) {
		sv[wave] = bv;
		si[wave] = bi;
	}
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int w = 1; w < LM_ARG_NT / WAVE; w++)
			if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) {
				bv = sv[w];
				bi = si[w];
			}
		/* no value above -inf (all NaN or -inf): index 0, as the loop of
		 * main.c leaves it */
		const int tok = bi == 0x7fffffff ? 0 : bi;
		st->tok = tok;
		if (tokens)
			tokens[st->step] = tok;
	}
}

/* the step's counters advance: step, pos, cache size */
__global__ void k_step_end(LmState *st)
{
	if (threadIdx.x == 0) {
		st->step += 1;
		st->pos += 1;
		st->size += 1;
	}
}

/* kvcache_rotate: rows [drop, drop + keep) of every (layer, kv head) move
 * to [0, keep); grid (rows of one move, heads * layers).  Reads all rows of
 * a (layer, head) slab before writing (rows are copied through registers
 * in order of the destination, so drop >= keep or a copy per row keeps
 * sources intact: the host guarantees drop >= keep or uses a staging
 * buffer). */
__global__ void k_kv_copy_rows(const float *__restrict__ src, float *__restrict__ dst,
			       size_t slab, size_t n)
{
	const size_t s = blockIdx.y;
	for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
	     i += (size_t)gridDim.x * blockDim.x)
		dst[s * slab + i] = src[s * slab + i];
}

/* ---------------------------------------------------------------------- */

extern "C" int lm_launch_embed(int wtype, const uint8_t *wte, int E, const LmState *st,
			       const int *prompt, float *hidden, void *stream)
{
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		hipLaunchKernelGGL(k_embed<1>, dim3(1), dim3(LM_NT), 0, s, wte, E, st, prompt, hidden);
	else if (wtype == 2)
		hipLaunchKernelGGL(k_embed<2>, dim3(1), dim3(LM_NT), 0, s, wte, E, st, prompt, hidden);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int lm_launch_add_rmsnorm(const float *a, const float *b, float *h, const float *w,
				     float *x, int E, void *stream)
{
	if (E < 1 || E > 32 * LM_NT)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(LM_NT), 0, (hipStream_t)stream, a, b, h, w,
			   x, E);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_qk_rope_kv(float *qkv, const float *q_norm, const float *k_norm,
				    const float *freq, const LmState *st, float *kc, float *vc,
				    int H, int KH, int HL, int C, void *stream)
{
	if (HL != LM_HLEN || KH < 1 || H % KH)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_qk_rope_kv, dim3(1), dim3(LM_NT), 0, (hipStream_t)stream, qkv, q_norm,
			   k_norm, freq, st, kc, vc, H, KH, HL, C);
	return (int)hipGetLastError();
}

extern "C" int lm_attn_chunks(int C, int window)
{
	const int span = window > 0 && window < C ? window : C;
	return (span + LM_CHUNK - 1) / LM_CHUNK;
}

extern "C" int lm_launch_attention(const float *q, const float *kc, const float *vc,
				   const LmState *st, float *part, float *out, int H, int KH,
				   int C, int window, float scale_div, void *stream)
{
	hipStream_t s = (hipStream_t)stream;
	const int nch = lm_attn_chunks(C, window);
	if (KH < 1 || H % KH)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_attn_part, dim3(H, nch), dim3(LM_NT), 0, s, q, kc, vc, st, part, H,
			   KH, C, window, scale_div);
	hipError_t e = hipGetLastError();
	if (e != hipSuccess)
		return (int)e;
	hipLaunchKernelGGL(k_attn_merge, dim3(H), dim3(LM_HLEN), 0, s, part, out, nch);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_argmax(const float *logits, int V, LmState *st, int *tokens,
				void *stream)
{
	hipLaunchKernelGGL(k_argmax, dim3(1), dim3(LM_ARG_NT), 0, (hipStream_t)stream, logits, V,
			   st, tokens);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_step_end(LmState *st, void *stream)
{
	hipLaunchKernelGGL(k_step_end, dim3(1), dim3(64), 0, (hipStream_t)stream, st);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_copy_rows(const float *src, float *dst, size_t slab, size_t n,
				   size_t slabs, void *stream)
{
	if (slabs == 0 || n == 0)
		return 0;
	hipLaunchKernelGGL(k_kv_copy_rows, dim3(64, (unsigned)slabs), dim3(256), 0,
			   (hipStream_t)stream, src, dst, slab, n);
	return (int)hipGetLastError();
}
