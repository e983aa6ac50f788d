/*
 * Kernels of the whole-model decode step around the MoE layer (hip_lm.c),
 * four launches per layer plus one for the head:
 *
 *   k_lm_qkv      the residual add (tensor_add, tensor.c:334-353) or the
 *                 token's embedding row (tensor_pick_rows, tensor.c:263-294),
 *                 rms_norm (nn.c:8-51) into LDS by every workgroup, then the
 *                 one-token product with the stacked [q; k; v] matrix
 *                 (olmoe.c:448-450)
 *   k_lm_attn     one (kv head, chunk of cache positions): the full-vector
 *                 RMSNorm of q and k (olmoe.c:454-458), RoPE on consecutive
 *                 pairs (rope_apply, nn.c:192-219), the new k/v row into the
 *                 cache (olmoe.c:240-262), then scores / sqrt(HLEN), the
 *                 chunk's max, exp-sum and exp-weighted v; the last chunk of
 *                 a head to finish merges the chunks into softmax . V
 *                 (olmoe.c:296-320, flash-decoding form)
 *   k_lm_oproj    the output product with the residual as its add operand
 *                 (olmoe.c:476-478); where the MoE launch does not take the
 *                 pre-MoE rms_norm (olmoe.c:482) itself, workgroup 0
 *                 gathers the rows and computes it
 *   k_lm_head     the residual add and the final rms_norm into LDS, the
 *                 lm_head product (olmoe.c:558-564), and the greedy pick
 *                 (main.c:189-193, the first maximum) by workgroup 0, which
 *                 also advances the step's counters
 *
 * The several-sequence and K-quant steps also use k_lm_norm_rows (residual
 * add and rms_norm of whole rows), k_lm_norm_parts (a matrix-core product's
 * partial sums, the residual and rms_norm in one launch), k_lm_pick_rows
 * and k_lm_embed.
 *
 * Every kernel reads the step's token, position and cache row from the
 * device state block (LmState), so one captured HIP graph serves every step.
 *
 * Results that one workgroup gathers from the others (attention partials,
 * the output product's rows, the workgroups' best logits) travel as 64-bit
 * words tagged with the step's epoch and the layer, written with
 * device-coherent stores and polled with device-coherent loads: no fence,
 * no reliance on store order.  The attention chunks of a head pick the
 * last of them with a counter (relaxed device atomics), reset by it; the
 * one-token products, whose grids the host sizes to be resident at once,
 * leave the gather to workgroup 0, which polls the words as they land.
 * Every poll is bounded; one that runs out sets LmState.err, which the
 * host reports.
 *
 * Compiled with -ffp-contract=off: fused multiply-adds only where written.
 */
#include "moe_qgemv.h"
#include "lm_internal.h"

#define LM_NT (QG_WAVES * WAVE) /* threads of every kernel here */
#define LM_SPIN (1 << 22)       /* poll rounds of a gather before it gives up */

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

/* the tag of gather `slot` (a layer, or LM_HEAD_SLOT) in this step */
__device__ static inline u32 lm_tag(const LmState *st, int slot)
{
	return (u32)st->epoch * LM_TAG_SLOTS + (u32)slot;
}

__device__ static inline uint64_t tagged(u32 tag, float v)
{
	return ((uint64_t)tag << 32) | __builtin_bit_cast(u32, v);
}

/* poll p until its tag is `tag`; its value, or 0 and the error word set */
__device__ static inline u32 poll_tag(const uint64_t *p, u32 tag, LmState *st)
{
	int step = 0;
	for (int round = 0;; round++) {
		const uint64_t v = ld_dev_u64(p);
		if ((u32)(v >> 32) == tag)
			return (u32)v;
		if (round >= LM_SPIN) {
			st_dev_u32((u32 *)&st->err, LM_ERR_GATHER);
			return 0;
		}
		backoff(step);
	}
}

/* v[i] = the value of p[i * stride] for the thread's entries i = tid,
 * tid + LM_NT, ... < n, its loads issued eight at a time before any is
 * checked; a late entry is polled on its own.  fn(i, value) consumes them. */
template <class Fn>
__device__ static inline void gather_tagged(const uint64_t *p, size_t stride, int n, u32 tag,
					    LmState *st, Fn fn)
{
	for (int i0 = threadIdx.x; i0 < n; i0 += 8 * LM_NT) {
		uint64_t v[8];
#pragma unroll
		for (int u = 0; u < 8; u++) {
			const int i = i0 + u * LM_NT;
			v[u] = i < n ? ld_dev_u64(&p[(size_t)i * stride]) : 0;
		}
#pragma unroll
		for (int u = 0; u < 8; u++) {
			const int i = i0 + u * LM_NT;
			if (i < n)
				fn(i, (u32)(v[u] >> 32) == tag ? (u32)v[u]
							       : poll_tag(&p[(size_t)i * stride], tag, st));
		}
	}
}

/* the last of n workgroups to arrive at counter *cnt (which it resets) */
__device__ static inline bool last_to_arrive(u32 *cnt, u32 n, int *s_flag)
{
	__syncthreads(); /* every thread's tagged stores are issued */
	if (threadIdx.x == 0) {
		const u32 old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED,
						       __HIP_MEMORY_SCOPE_AGENT);
		*s_flag = old == n - 1;
		if (old == n - 1)
			__hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
	}
	__syncthreads();
	return *s_flag != 0;
}

/* the step's token: the prompt's while it lasts, then the last pick */
__device__ static inline int step_token(const LmState *st, const int *prompt)
{
	return st->step < st->n_prompt ? prompt[st->step] : st->tok;
}

/* four consecutive values (float4 index c4) of a dequantized row:
 * d * q (quant.c:157-196) */
template <int WT>
__device__ static inline float4 dequant4(const uint8_t *row, int c4)
{
	constexpr int BB = WT == 1 ? 34 : 18;
	const uint8_t *b = row + (size_t)(c4 / 8) * BB;
	const float d = f16_bits_to_f32((u32)b[0] | ((u32)b[1] << 8));
	const int j = (c4 % 8) * 4;
	float q[4];
#pragma unroll
	for (int u = 0; u < 4; u++) {
		if (WT == 1)
			q[u] = (float)(int8_t)b[2 + j + u];
		else
			q[u] = (float)((j < 16 ? (b[2 + j + u] & 15) : (b[2 + j + u - 16] >> 4)) - 8);
	}
	return make_float4(d * q[0], d * q[1], d * q[2], d * q[3]);
}

/*
 * Every workgroup puts x = rms_norm(v) * w into LDS (segment layout) with
 * v = a + b (b may be NULL), or v = the dequantized row `emb`.  h_out (one
 * workgroup passes it) receives v.  rms = sqrtf(sum(v^2) / E + 1e-5f),
 * x = (v / rms) * w, as nn.c:8-51.
 */
template <int WT>
__device__ static void stage_norm(float *sx, float *red, int E, const float *a, const float *b,
				  const uint8_t *emb, const float *w, float *h_out)
{
	/* NB float4s of a thread in flight at once (a loop that loaded one per
	 * iteration waited a round trip each: h_out may alias a and b); w stays
	 * in registers when one batch covers E */
	constexpr int NB = 4;
	const int n4 = E / 4;
	const bool one = n4 <= NB * LM_NT;
	float4 wv[NB];
	float ss = 0.0f;
	for (int c0 = threadIdx.x; c0 < n4; c0 += NB * LM_NT) {
		float4 v[NB], u[NB];
#pragma unroll
		for (int k = 0; k < NB; k++) {
			const int c4 = c0 + k * LM_NT;
			if (c4 >= n4)
				break;
			if (emb) {
				v[k] = dequant4<WT>(emb, c4);
			} else {
				v[k] = ((const float4 *)a)[c4];
				if (b)
					u[k] = ((const float4 *)b)[c4];
			}
			if (one)
				wv[k] = ((const float4 *)w)[c4];
		}
#pragma unroll
		for (int k = 0; k < NB; k++) {
			const int c4 = c0 + k * LM_NT;
			if (c4 >= n4)
				break;
			if (!emb && b) {
				v[k].x = v[k].x + u[k].x;
				v[k].y = v[k].y + u[k].y;
				v[k].z = v[k].z + u[k].z;
				v[k].w = v[k].w + u[k].w;
			}
			if (h_out)
				((float4 *)h_out)[c4] = v[k];
			*(float4 *)(sx + (c4 >> 4) * SEG_STRIDE + (c4 & 15) * 4) = v[k];
			const float q0 = v[k].x * v[k].x, q1 = v[k].y * v[k].y;
			const float q2 = v[k].z * v[k].z, q3 = v[k].w * v[k].w;
			ss = ss + q0;
			ss = ss + q1;
			ss = ss + q2;
			ss = ss + q3;
		}
	}
	const float rms = sqrtf(block_sum(ss, red) / (float)E + 1e-5f);
	for (int c0 = threadIdx.x; c0 < n4; c0 += NB * LM_NT) {
		if (!one) {
#pragma unroll
			for (int k = 0; k < NB; k++) {
				const int c4 = c0 + k * LM_NT;
				if (c4 < n4)
					wv[k] = ((const float4 *)w)[c4];
			}
		}
#pragma unroll
		for (int k = 0; k < NB; k++) {
			const int c4 = c0 + k * LM_NT;
			if (c4 >= n4)
				break;
			float4 *p = (float4 *)(sx + (c4 >> 4) * SEG_STRIDE + (c4 & 15) * 4);
			float4 v = *p;
			v.x = (v.x / rms) * wv[k].x;
			v.y = (v.y / rms) * wv[k].y;
			v.z = (v.z / rms) * wv[k].z;
			v.w = (v.w / rms) * wv[k].w;
			*p = v;
		}
	}
	__syncthreads();
}

/* ---------------------------------------------------------------------- */
/* k_lm_qkv                                                               */
/* ---------------------------------------------------------------------- */

/* qkv = rms_norm(src) * w . Wqkv^T; src = a + b, or the step's token row of
 * wte when a is NULL; workgroup 0 writes src to h_out */
template <int WT, int C>
__global__ __launch_bounds__(LM_NT) __attribute__((amdgpu_waves_per_eu(4)))
void k_lm_qkv(const uint8_t *__restrict__ W, size_t rb, int N, int K, const float *a,
	      const float *b, const float *__restrict__ w, float *h_out,
	      const uint8_t *__restrict__ wte, const LmState *__restrict__ st,
	      const int *__restrict__ prompt, float *__restrict__ out)
{
	extern __shared__ __attribute__((aligned(16))) float sx[];
	__shared__ float red[LM_NT / WAVE];
	constexpr int BB = WT == 1 ? 34 : 18;
	const uint8_t *emb =
		a ? nullptr : wte + (size_t)step_token(st, prompt) * (size_t)(K / 32) * BB;
	stage_norm<WT>(sx, red, K, a, b, emb, w, blockIdx.x == 0 ? h_out : nullptr);
	qgemv_body<WT, C, true, true>(sx, W, rb, N, K, nullptr, 1, 1, nullptr, 0, out);
}

/* ---------------------------------------------------------------------- */
/* k_lm_attn                                                              */
/* ---------------------------------------------------------------------- */

/*
 * Scores are q . k / scale (OLMoE's tensor_div_scalar by sqrt(HLEN),
 * olmoe.c:295) or q . k * scale (Mixtral's flash_attention, scale =
 * 1 / sqrt(HLEN), nn.c:578) as scale_mul says.
 *
 * Grid (KH, nact, sequences): nact = the chunks of LM_CHUNK rows that cover
 * the cache rows [lo, AT), AT = size + 1 (lo > 0 past a sliding window),
 * which the host knows for every step.  Workgroup (kh, c) takes the G = H /
 * KH query heads of kv head kh (grouped-query attention, llama.c:286-288:
 * head h reads kv head h / G) over rows [j0, j0 + n), so each k and v row
 * is read once for its G heads; the row `size` is this step's k and v,
 * which the chunk holding it takes from LDS (and writes to the cache).
 * The cached k and v rows of the chunk are loaded as soon as the cache size
 * is known, so they arrive while q and k are normalised and rotated.
 * Scores: 4 threads per position, 32 dims each, all G heads from one read
 * of the row; softmax: wave g % NW takes head g (lane = position); v sums:
 * one dim per thread over half the positions, G heads from one read.  One
 * chunk writes out[h] = o / l itself; with more, partials part[h][c] =
 * {m, l, o[HL]} (stride nstride chunks) go out tagged, and one of kv head
 * kh's chunks (chunk 0 where the grid is resident at once, else the last
 * to count in) merges its G heads: out[h][d] = sum_c exp(m_c - M)
 * o_c[d] / sum_c exp(m_c - M) l_c.  Every head's arithmetic is the same
 * whatever G.
 */
template <int G, int PF>
__global__ __launch_bounds__(LM_NT) void k_lm_attn(const float *__restrict__ qkv,
						   const float *__restrict__ q_norm,
						   const float *__restrict__ k_norm,
						   const float *__restrict__ freq, LmState *st,
						   float *__restrict__ kc, float *__restrict__ vc,
						   uint64_t *part, u32 *cnt, float *__restrict__ out,
						   int H, int KH, int C, int window, float scale,
						   int scale_mul, int layer, int nstride, size_t cstride)
{
	constexpr int HL = LM_HLEN, CH = LM_CHUNK, NW = LM_NT / WAVE;
	__shared__ float cs[HL / 2], sn[HL / 2], sq[G][HL], sk[HL], sv[HL], sp[G][CH];
	__shared__ float so[G][LM_NT];
	__shared__ float red[NW];
	__shared__ float s_f[G][LM_MAX_CHUNKS], s_l[G][LM_MAX_CHUNKS];
	__shared__ float s_m[G], s_sum[G];
	__shared__ int s_flag;
	const int kh = blockIdx.x, c = blockIdx.y, nact = gridDim.y;
	const int h0 = kh * G; /* the group's first query head */
	const int EQ = H * HL, EK = KH * HL;
	{ /* sequence blockIdx.z of several decoding in lockstep: its q/k/v row,
	   * cache, partials, counters and output row */
		const size_t sq = blockIdx.z;
		qkv += sq * (size_t)(EQ + 2 * EK);
		kc += sq * cstride;
		vc += sq * cstride;
		part += sq * (size_t)H * nstride * (HL + 2);
		cnt += sq * (size_t)H;
		out += sq * (size_t)EQ;
	}
	const float *q = qkv, *k = qkv + EQ, *v = qkv + EQ + EK;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;

	/* every load that does not depend on the counters goes out first */
	float qx[G], qw[G], kx = 0.0f, vx = 0.0f, kw = 1.0f, fr = 0.0f;
#pragma unroll
	for (int g = 0; g < G; g++) {
		qx[g] = 0.0f;
		qw[g] = 1.0f;
	}
	if (tid < HL) {
#pragma unroll
		for (int g = 0; g < G; g++)
			qx[g] = q[(h0 + g) * HL + tid];
		kx = k[kh * HL + tid];
		vx = v[kh * HL + tid];
		if (q_norm) {
#pragma unroll
			for (int g = 0; g < G; g++)
				qw[g] = q_norm[(h0 + g) * HL + tid];
			kw = k_norm[kh * HL + tid];
		}
	}
	if (tid < HL / 2)
		fr = freq[tid];
	float s1 = 0.0f, s2 = 0.0f;
	if (q_norm) {
		/* eight q and eight k loads in flight (rows clamped: no branch per
		 * load), each sum added in index order; one loop, so the k loads
		 * do not wait behind the q sums (two loops took two round trips) */
		for (int i0 = tid; i0 < max(EQ, EK); i0 += 8 * LM_NT) {
			float qv[8], kv[8];
#pragma unroll
			for (int u = 0; u < 8; u++) {
				qv[u] = q[min(i0 + u * LM_NT, EQ - 1)];
				kv[u] = k[min(i0 + u * LM_NT, EK - 1)];
			}
#pragma unroll
			for (int u = 0; u < 8; u++)
				if (i0 + u * LM_NT < EQ) {
					const float t = qv[u] * qv[u];
					s1 = s1 + t;
				}
#pragma unroll
			for (int u = 0; u < 8; u++)
				if (i0 + u * LM_NT < EK) {
					const float t = kv[u] * kv[u];
					s2 = s2 + t;
				}
		}
	}
	const int size = st->size, spos = st->pos;
	const u32 tag = lm_tag(st, layer);
	const int AT = size + 1;
	const int lo = window > 0 && AT > window ? AT - window : 0;
	const int j0 = lo + c * CH;
	const int n = max(0, min(CH, AT - j0));
	/* olmoe_decode: a position past the context is the cache size
	 * (olmoe.c:514-515) */
	const int pos = spos < C ? spos : size;
	const int jn = size - j0; /* the new row's place in this chunk, if 0 <= jn < n */
	const float *K = kc + ((size_t)kh * C + j0) * HL, *V = vc + ((size_t)kh * C + j0) * HL;
	/* the chunk's cached k and v rows (all but the new one): thread (j =
	 * tid / 4, d0) takes 32 dims of row j's k; thread (d, half) dim d of
	 * rows half, half + 2, ... of v.  PF: they go out now, to arrive while
	 * q and k are normalised and rotated (3 waves per SIMD instead of 7,
	 * for grids that fit the device at once) */
	const int jq = tid / 4, d0 = (tid % 4) * 32;
	const int dv = tid % HL, half = tid / HL;
	float kr[32], vr[CH / (LM_NT / HL)];
	auto load_k = [&]() {
		if (jq < n && jq != jn) {
			const float4 *k4 = (const float4 *)(K + (size_t)jq * HL + d0);
#pragma unroll
			for (int u = 0; u < 8; u++) {
				const float4 kv = k4[u];
				kr[4 * u + 0] = kv.x;
				kr[4 * u + 1] = kv.y;
				kr[4 * u + 2] = kv.z;
				kr[4 * u + 3] = kv.w;
			}
		}
	};
	/* every load unconditional, its row clamped into [0, n - 1] (rows of the
	 * cache: every launched chunk has j0 < AT, so n >= 1): rows past n and
	 * the new row jn are loaded but never used (the sums below stop at n
	 * and take row jn from LDS); one branch per load had cost a wave ~2 us
	 * of issue */
	auto load_v = [&]() {
		const int nc = max(n, 1);
#pragma unroll
		for (int i = 0; i < CH / (LM_NT / HL); i++) {
			const int j = min(half + i * (LM_NT / HL), nc - 1);
			vr[i] = V[(size_t)j * HL + dv];
		}
	};
	if constexpr (PF >= 1)
		load_k();
	if constexpr (PF >= 2)
		load_v();

	if (tid < HL / 2) {
		const float ang = (float)pos * fr;
		cs[tid] = cosf(ang);
		sn[tid] = sinf(ang);
	}
	if (q_norm) {
		const float rq = sqrtf(block_sum(s1, red) / (float)EQ + 1e-5f);
		const float rk = sqrtf(block_sum(s2, red) / (float)EK + 1e-5f);
#pragma unroll
		for (int g = 0; g < G; g++) {
			const float r = qx[g] / rq;
			qx[g] = r * qw[g];
		}
		const float t = kx / rk;
		kx = t * kw;
	}
	if (tid < HL) {
#pragma unroll
		for (int g = 0; g < G; g++)
			sq[g][tid] = qx[g];
		sk[tid] = kx;
		sv[tid] = vx;
	}
	__syncthreads();
	/* x0' = x0 cos - x1 sin, x1' = x0 sin + x1 cos (one FMA each): pair i
	 * of head g is item g * HL / 2 + i, k's the last HL / 2 items */
	for (int it = tid; it < (G + 1) * (HL / 2); it += LM_NT) {
		const int g = it / (HL / 2), i = it % (HL / 2);
		float *x = g < G ? sq[g] : sk;
		const float co = cs[i], si = sn[i];
		const float x0 = x[2 * i], x1 = x[2 * i + 1];
		x[2 * i] = __builtin_fmaf(x0, co, -(x1 * si));
		x[2 * i + 1] = __builtin_fmaf(x0, si, x1 * co);
	}
	__syncthreads();
	if (jn >= 0 && jn < n && tid < HL) {
		kc[((size_t)kh * C + size) * HL + tid] = sk[tid];
		vc[((size_t)kh * C + size) * HL + tid] = sv[tid];
	}
	if constexpr (PF < 1)
		load_k();
	{
		const int j = jq;
		float acc[G];
#pragma unroll
		for (int g = 0; g < G; g++)
			acc[g] = 0.0f;
		if (j < n) {
			if (j == jn) {
#pragma unroll
				for (int u = 0; u < 32; u++)
					kr[u] = sk[d0 + u];
			}
#pragma unroll
			for (int g = 0; g < G; g++)
#pragma unroll
				for (int u = 0; u < 32; u++)
					acc[g] = __builtin_fmaf(sq[g][d0 + u], kr[u], acc[g]);
		}
#pragma unroll
		for (int g = 0; g < G; g++) {
			float a = acc[g];
			a += __shfl_xor(a, 1, WAVE);
			a += __shfl_xor(a, 2, WAVE);
			if (tid % 4 == 0)
				sp[g][j] = j < n ? (scale_mul ? a * scale : a / scale) : -INFINITY;
		}
	}
	__syncthreads();
	/* softmax of head g on wave g % NW, lane = position (the wave's xor
	 * trees: the same sums as a workgroup-wide reduction whose other waves
	 * add zeros) */
	for (int g = wave; g < G; g += NW) {
		float mv = sp[g][lane];
		for (int o2 = WAVE / 2; o2 > 0; o2 >>= 1)
			mv = fmaxf(mv, __shfl_xor(mv, o2, WAVE));
		const float e = lane < n ? moe_expf(sp[g][lane] - mv) : 0.0f;
		sp[g][lane] = e;
		float sv2 = e;
		for (int o2 = WAVE / 2; o2 > 0; o2 >>= 1)
			sv2 += __shfl_xor(sv2, o2, WAVE);
		if (lane == 0) {
			s_m[g] = mv;
			s_sum[g] = sv2;
		}
	}
	if constexpr (PF < 2)
		load_v();
	__syncthreads();
	{
		float o[G];
#pragma unroll
		for (int g = 0; g < G; g++)
			o[g] = 0.0f;
#pragma unroll
		for (int i = 0; i < CH / (LM_NT / HL); i++) {
			const int j = half + i * (LM_NT / HL);
			if (j >= n)
				break;
			const float vj = j == jn ? sv[dv] : vr[i];
#pragma unroll
			for (int g = 0; g < G; g++)
				o[g] = __builtin_fmaf(sp[g][j], vj, o[g]);
		}
#pragma unroll
		for (int g = 0; g < G; g++)
			so[g][tid] = o[g];
	}
	__syncthreads();
	float o[G];
	if (tid < HL) {
#pragma unroll
		for (int g = 0; g < G; g++) {
			o[g] = so[g][tid];
			for (int u = 1; u < LM_NT / HL; u++)
				o[g] += so[g][tid + u * HL];
		}
	}
	if (nact == 1) { /* the whole context in one chunk: no merge */
		if (tid < HL)
#pragma unroll
			for (int g = 0; g < G; g++)
				out[(h0 + g) * HL + tid] = o[g] / s_sum[g];
		return;
	}
#pragma unroll
	for (int g = 0; g < G; g++) {
		uint64_t *pp = part + ((size_t)(h0 + g) * nstride + c) * (HL + 2);
		if (tid < HL)
			st_dev_u64(&pp[2 + tid], tagged(tag, o[g]));
		if (tid == 0) {
			st_dev_u64(&pp[0], tagged(tag, n > 0 ? s_m[g] : -INFINITY));
			st_dev_u64(&pp[1], tagged(tag, s_sum[g]));
		}
	}
	/* PF 2 (the grid is resident at once): chunk 0 merges, polling the
	 * others' partials as they land; else the last chunk to count in */
	if constexpr (PF == 2) {
		if (c != 0)
			return;
	} else if (!last_to_arrive(&cnt[kh], (u32)nact, &s_flag)) {
		return;
	}
	/* merge the nact chunks of the G heads: every head's m and l in one
	 * batch of loads (a late one polled alone), then the o sums two heads
	 * at a time, sixteen chunks' loads in flight (merging the heads one
	 * after another took ~20 dependent round trips for 4 heads x 17
	 * chunks); each head's arithmetic in chunk order as before */
	const int NML = G * nact;
	for (int e0 = tid; e0 < NML; e0 += 8 * LM_NT) {
		uint64_t vm[8], vl[8];
#pragma unroll
		for (int u = 0; u < 8; u++) {
			const int e = e0 + u * LM_NT;
			const uint64_t *pe =
				part + ((size_t)(h0 + e / nact) * nstride + e % nact) * (HL + 2);
			vm[u] = e < NML ? ld_dev_u64(&pe[0]) : 0;
			vl[u] = e < NML ? ld_dev_u64(&pe[1]) : 0;
		}
#pragma unroll
		for (int u = 0; u < 8; u++) {
			const int e = e0 + u * LM_NT;
			if (e >= NML)
				break;
			const int g = e / nact, cc = e % nact;
			const uint64_t *pe = part + ((size_t)(h0 + g) * nstride + cc) * (HL + 2);
			const u32 mb = (u32)(vm[u] >> 32) == tag ? (u32)vm[u] : poll_tag(&pe[0], tag, st);
			const u32 lb = (u32)(vl[u] >> 32) == tag ? (u32)vl[u] : poll_tag(&pe[1], tag, st);
			s_f[g][cc] = __builtin_bit_cast(float, mb);
			s_l[g][cc] = __builtin_bit_cast(float, lb);
		}
	}
	__syncthreads();
	/* head g's maximum M on wave g % NW (max: any order), then its weights
	 * exp(m_c - M) (0 for an empty chunk) */
	for (int g = wave; g < G; g += NW) {
		float M = -INFINITY;
		for (int cc = lane; cc < nact; cc += WAVE)
			M = fmaxf(M, s_f[g][cc]);
		for (int o2 = WAVE / 2; o2 > 0; o2 >>= 1)
			M = fmaxf(M, __shfl_xor(M, o2, WAVE));
		for (int cc = lane; cc < nact; cc += WAVE)
			s_f[g][cc] = s_l[g][cc] > 0.0f ? moe_expf(s_f[g][cc] - M) : 0.0f;
	}
	__syncthreads();
	{
		constexpr int HPR = LM_NT / HL; /* heads merged at once */
		const int d = tid % HL;
		for (int g = tid / HL; g < G; g += HPR) {
			const uint64_t *ph = part + (size_t)(h0 + g) * nstride * (HL + 2);
			float L = 0.0f, acc = 0.0f;
			for (int c0 = 0; c0 < nact; c0 += 16) {
				uint64_t vv[16];
#pragma unroll
				for (int u = 0; u < 16; u++)
					vv[u] = c0 + u < nact
							? ld_dev_u64(&ph[(size_t)(c0 + u) * (HL + 2) + 2 + d])
							: 0;
#pragma unroll
				for (int u = 0; u < 16; u++) {
					const int cc = c0 + u;
					if (cc >= nact)
						break;
					const u32 ob =
						(u32)(vv[u] >> 32) == tag
							? (u32)vv[u]
							: poll_tag(&ph[(size_t)cc * (HL + 2) + 2 + d], tag, st);
					const float f = s_f[g][cc];
					L = __builtin_fmaf(f, s_l[g][cc], L);
					acc = __builtin_fmaf(f, __builtin_bit_cast(float, ob), acc);
				}
			}
			out[(h0 + g) * HL + d] = acc / L;
		}
	}
}

/* ---------------------------------------------------------------------- */
/* k_lm_oproj                                                             */
/* ---------------------------------------------------------------------- */

/*
 * out[E] = add + x . Wo^T (the residual stream after attention), each row
 * also stored tagged in rows_t; workgroup 0 reads them all back and writes
 * x_out = rms_norm(out) * w (the MoE layer's input).  x_out NULL: the
 * product alone (the MoE launch normalises out itself).
 */
template <int WT, int C>
__global__ __launch_bounds__(LM_NT) __attribute__((amdgpu_waves_per_eu(4)))
void k_lm_oproj(const uint8_t *__restrict__ W, size_t rb, int N, int K,
		const float *__restrict__ x, const float *__restrict__ add, float *__restrict__ out,
		uint64_t *rows_t, const float *__restrict__ w, float *__restrict__ x_out,
		LmState *st, int layer)
{
	extern __shared__ __attribute__((aligned(16))) float sx[];
	__shared__ float red[LM_NT / WAVE];
	if (!x_out) {
		qgemv_body<WT, C, true>(sx, W, rb, N, K, x, 1, 1, add, 0, out, QgNoHook{});
		return;
	}
	const u32 tag = lm_tag(st, layer);
	auto hook = [=](int row, float r) { st_dev_u64(&rows_t[row], tagged(tag, r)); };
	qgemv_body<WT, C, true>(sx, W, rb, N, K, x, 1, 1, add, 0, out, hook);
	/* workgroup 0 normalises, polling the rows as they land: the host sizes
	 * the grid to be resident at once, so every row comes (counting the
	 * workgroups in at device counters put 2-3 us of atomics behind the
	 * slowest one) */
	if (blockIdx.x != 0)
		return;
	/* the norm weights of this thread's outputs, WB at a time, the first
	 * batch loading while the rows are gathered (a loop of one load per
	 * output waited a round trip each) */
	constexpr int WB = 16;
	float wv[WB];
	auto load_w = [&](int i0) {
#pragma unroll
		for (int k = 0; k < WB; k++) {
			const int i = i0 + k * LM_NT;
			wv[k] = i < N ? w[i] : 0.0f;
		}
	};
	load_w(threadIdx.x);
	float ss = 0.0f;
	gather_tagged(rows_t, 1, N, tag, st, [&](int i, u32 b) {
		const float v = __builtin_bit_cast(float, b);
		sx[i] = v;
		const float t = v * v;
		ss = ss + t;
	});
	const float rms = sqrtf(block_sum(ss, red) / (float)N + 1e-5f);
	for (int i0 = threadIdx.x; i0 < N; i0 += WB * LM_NT) {
		if (i0 != (int)threadIdx.x)
			load_w(i0);
#pragma unroll
		for (int k = 0; k < WB; k++) {
			const int i = i0 + k * LM_NT;
			if (i < N) {
				const float r = sx[i] / rms;
				x_out[i] = r * wv[k];
			}
		}
	}
}

/* ---------------------------------------------------------------------- */
/* k_lm_head                                                              */
/* ---------------------------------------------------------------------- */

__device__ static inline void better(float &bv, int &bi, float v, int i)
{
	if (v > bv || (v == bv && i < bi)) {
		bv = v;
		bi = i;
	}
}

/*
 * logits[V] = rms_norm(a + b) * w . lm_head^T; every workgroup's first
 * maximum goes out tagged, and the last workgroup picks the first maximum
 * of all (main.c:189-193), writes it as the next token and tokens[step],
 * and advances the counters (olmoe_generate: model->pos++, the cache row,
 * the step and the epoch).
 */
template <int WT, int C>
__global__ __launch_bounds__(LM_NT) __attribute__((amdgpu_waves_per_eu(4)))
void k_lm_head(const uint8_t *__restrict__ W, size_t rb, int N, int K, const float *a,
	       const float *b, const float *__restrict__ w, float *__restrict__ out,
	       uint64_t *best, LmState *st, int *tokens)
{
	extern __shared__ __attribute__((aligned(16))) float sx[];
	__shared__ float red[LM_NT / WAVE];
	__shared__ float s_v[LM_NT / WAVE];
	__shared__ int s_i[LM_NT / WAVE];
	const u32 tag = lm_tag(st, LM_HEAD_SLOT);
	stage_norm<WT>(sx, red, K, a, b, nullptr, w, nullptr);
	float bv = -INFINITY;
	int bi = 0x7fffffff;
	auto hook = [&](int row, float r) { better(bv, bi, r, row); };
	qgemv_body<WT, C, true, true>(sx, W, rb, N, K, nullptr, 1, 1, nullptr, 0, out, hook);
	for (int o = WAVE / 2; o > 0; o >>= 1)
		better(bv, bi, __shfl_xor(bv, o, WAVE), __shfl_xor(bi, o, WAVE));
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	if (lane == 0) {
		s_v[wave] = bv;
		s_i[wave] = bi;
	}
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int u = 1; u < LM_NT / WAVE; u++)
			better(bv, bi, s_v[u], s_i[u]);
		st_dev_u64(&best[2 * blockIdx.x], tagged(tag, bv));
		st_dev_u64(&best[2 * blockIdx.x + 1], ((uint64_t)tag << 32) | (u32)bi);
	}
	/* workgroup 0 picks, polling the workgroups' bests as they land (the
	 * grid is resident at once; every workgroup read the epoch before its
	 * tagged best, so advancing it after all of them is safe) */
	if (blockIdx.x != 0)
		return;
	bv = -INFINITY;
	bi = 0x7fffffff;
	/* entries 2g (value) and 2g + 1 (index) of workgroup g */
	__shared__ float s_bv[LM_MAX_HEAD_WG];
	gather_tagged(best, 2, (int)gridDim.x, tag, st,
		      [&](int g, u32 b) { s_bv[g] = __builtin_bit_cast(float, b); });
	gather_tagged(best + 1, 2, (int)gridDim.x, tag, st,
		      [&](int g, u32 b) { better(bv, bi, s_bv[g], (int)b); });
	for (int o = WAVE / 2; o > 0; o >>= 1)
		better(bv, bi, __shfl_xor(bv, o, WAVE), __shfl_xor(bi, o, WAVE));
	if (lane == 0) {
		s_v[wave] = bv;
		s_i[wave] = bi;
	}
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int u = 1; u < LM_NT / WAVE; u++)
			better(bv, bi, s_v[u], s_i[u]);
		/* no value above -inf (all NaN): index 0, as main.c's loop leaves it */
		const int tok = bi == 0x7fffffff ? 0 : bi;
		st->tok = tok;
		if (tokens)
			tokens[st->step] = tok;
		st->step += 1;
		st->pos += 1;
		st->size += 1;
		st->epoch += 1;
	}
}

/* the step's counters advance (a step without the lm_head) */
__global__ void k_lm_step_end(LmState *st)
{
	if (threadIdx.x == 0) {
		st->step += 1;
		st->pos += 1;
		st->size += 1;
		st->epoch += 1;
	}
}

/* kvcache_rotate's moves: dst[s * slab + i] = src[s * slab + i] */
__global__ void k_lm_copy_rows(const float *__restrict__ src, float *__restrict__ dst,
			       size_t slab, size_t n)
{
	const size_t s = blockIdx.y;
	for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
	     i += (size_t)gridDim.x * blockDim.x)
		dst[s * slab + i] = src[s * slab + i];
}

/* ---------------------------------------------------------------------- */
/* several sequences in lockstep                                          */
/* ---------------------------------------------------------------------- */

/*
 * Workgroup s, sequence s: v = a[s] + b[s] (b may be NULL), or the
 * embedding row of the sequence's step token when a is NULL (the prompt's,
 * prompt[s][step], while it lasts, then its last pick btok[s]); h_out[s]
 * receives v (may be NULL), x_out[s] = rms_norm(v) * w.
 */
template <int WT>
__global__ __launch_bounds__(LM_NT) void k_lm_norm_rows(int E, const float *a, const float *b,
							const float *__restrict__ w, float *h_out,
							float *__restrict__ x_out,
							const uint8_t *__restrict__ wte,
							const LmState *__restrict__ st,
							const int *__restrict__ prompt,
							const int *__restrict__ btok)
{
	extern __shared__ __attribute__((aligned(16))) float sx[];
	__shared__ float red[LM_NT / WAVE];
	constexpr int BB = WT == 1 ? 34 : 18;
	const int s = blockIdx.x;
	const size_t o = (size_t)s * E;
	const uint8_t *emb = nullptr;
	if (!a) {
		const int tok = st->step < st->n_prompt
					? prompt[(size_t)s * st->n_prompt + st->step]
					: btok[s];
		emb = wte + (size_t)tok * (size_t)(E / 32) * BB;
	}
	stage_norm<WT>(sx, red, E, a ? a + o : nullptr, b ? b + o : nullptr, emb, w,
		       h_out ? h_out + o : nullptr);
	for (int c4 = threadIdx.x; c4 < E / 4; c4 += LM_NT)
		((float4 *)(x_out + o))[c4] =
			*(const float4 *)(sx + (c4 >> 4) * SEG_STRIDE + (c4 & 15) * 4);
}

/*
 * Row s of h = add + the KS partial sums of a matrix-core product (slices
 * of TN floats, added in stretch order after the first, then added to add:
 * k_qmm_reduce's arithmetic) into h_out, then x_out = rms_norm(h) * w with
 * stage_norm's arithmetic (the thread's float4s in order, the four squares
 * of each, block_sum, (h / rms) * w): one launch where the product's
 * reduce and the row norm were two, with the same bits.
 */
__global__ __launch_bounds__(LM_NT) void k_lm_norm_parts(int E, const float *__restrict__ part,
							 int KS, size_t TN,
							 const float *__restrict__ add,
							 const float *__restrict__ w,
							 float *__restrict__ h_out,
							 float *__restrict__ x_out)
{
	extern __shared__ __attribute__((aligned(16))) float sx[];
	__shared__ float red[LM_NT / WAVE];
	constexpr int NB = 4;
	const size_t o = (size_t)blockIdx.x * E;
	const int n4 = E / 4;
	const float4 *p4 = (const float4 *)(part + o), *a4 = (const float4 *)(add + o);
	const size_t ts = TN / 4; /* float4s between slices */
	float ss = 0.0f;
	for (int c0 = threadIdx.x; c0 < n4; c0 += NB * LM_NT) {
		/* the slices' loads in batches of 8, all of a batch before its adds */
		float4 v[NB], a[NB];
#pragma unroll
		for (int k = 0; k < NB; k++) {
			const int c4 = min(c0 + k * LM_NT, n4 - 1);
			v[k] = p4[c4];
			a[k] = a4[c4];
		}
		for (int z0 = 1; z0 < KS; z0 += 8) {
			float4 q[NB][8];
#pragma unroll
			for (int k = 0; k < NB; k++)
#pragma unroll
				for (int u = 0; u < 8; u++)
					q[k][u] = p4[(size_t)min(z0 + u, KS - 1) * ts +
						     min(c0 + k * LM_NT, n4 - 1)];
#pragma unroll
			for (int k = 0; k < NB; k++)
#pragma unroll
				for (int u = 0; u < 8; u++)
					if (z0 + u < KS) {
						v[k].x += q[k][u].x;
						v[k].y += q[k][u].y;
						v[k].z += q[k][u].z;
						v[k].w += q[k][u].w;
					}
		}
#pragma unroll
		for (int k = 0; k < NB; k++) {
			v[k].x = a[k].x + v[k].x;
			v[k].y = a[k].y + v[k].y;
			v[k].z = a[k].z + v[k].z;
			v[k].w = a[k].w + v[k].w;
		}
#pragma unroll
		for (int k = 0; k < NB; k++) {
			const int c4 = c0 + k * LM_NT;
			if (c4 >= n4)
				break;
			((float4 *)(h_out + o))[c4] = v[k];
			((float4 *)sx)[c4] = v[k];
			const float q0 = v[k].x * v[k].x, q1 = v[k].y * v[k].y;
			const float q2 = v[k].z * v[k].z, q3 = v[k].w * v[k].w;
			ss = ss + q0;
			ss = ss + q1;
			ss = ss + q2;
			ss = ss + q3;
		}
	}
	const float rms = sqrtf(block_sum(ss, red) / (float)E + 1e-5f);
	for (int c4 = threadIdx.x; c4 < n4; c4 += LM_NT) {
		float4 v = ((const float4 *)sx)[c4];
		const float4 wv = ((const float4 *)w)[c4];
		v.x = (v.x / rms) * wv.x;
		v.y = (v.y / rms) * wv.y;
		v.z = (v.z / rms) * wv.z;
		v.w = (v.w / rms) * wv.w;
		((float4 *)(x_out + o))[c4] = v;
	}
}

/* workgroup s: the first maximum of logits[s] (main.c:189-193) becomes the
 * sequence's next token btok[s] and tokens[s * tstride + step] */
#define PK_NT 1024 /* threads of the pick: a 50304-entry row in one round of loads */

__global__ __launch_bounds__(PK_NT) void k_lm_pick_rows(const float *__restrict__ logits,
							int V, const LmState *__restrict__ st,
							int *__restrict__ btok, int *tokens,
							int tstride)
{
	__shared__ float s_v[PK_NT / WAVE];
	__shared__ int s_i[PK_NT / WAVE];
	const float *row = logits + (size_t)blockIdx.x * V;
	float bv = -INFINITY;
	int bi = 0x7fffffff;
	/* sixteen loads in flight per thread, 16-byte ones where the rows are
	 * 16-byte aligned (V % 4 == 0; a single workgroup of 256 threads
	 * with 4-byte loads took ~22 us for 50304 logits); better() does not
	 * depend on the order */
	if ((V & 3) == 0) {
		const float4 *r4 = (const float4 *)row;
		const int n4 = V / 4;
		for (int i0 = threadIdx.x; i0 < n4; i0 += 16 * PK_NT) {
			float4 v[16];
#pragma unroll
			for (int u = 0; u < 16; u++)
				v[u] = r4[min(i0 + u * PK_NT, n4 - 1)];
#pragma unroll
			for (int u = 0; u < 16; u++) {
				const int c = i0 + u * PK_NT;
				if (c < n4) {
					better(bv, bi, v[u].x, 4 * c);
					better(bv, bi, v[u].y, 4 * c + 1);
					better(bv, bi, v[u].z, 4 * c + 2);
					better(bv, bi, v[u].w, 4 * c + 3);
				}
			}
		}
	} else {
		for (int i0 = threadIdx.x; i0 < V; i0 += 16 * PK_NT) {
			float v[16];
#pragma unroll
			for (int u = 0; u < 16; u++)
				v[u] = row[min(i0 + u * PK_NT, V - 1)];
#pragma unroll
			for (int u = 0; u < 16; u++)
				if (i0 + u * PK_NT < V)
					better(bv, bi, v[u], i0 + u * PK_NT);
		}
	}
	for (int o = WAVE / 2; o > 0; o >>= 1)
		better(bv, bi, __shfl_xor(bv, o, WAVE), __shfl_xor(bi, o, WAVE));
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	if (lane == 0) {
		s_v[wave] = bv;
		s_i[wave] = bi;
	}
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int u = 1; u < PK_NT / WAVE; u++)
			better(bv, bi, s_v[u], s_i[u]);
		/* no value above -inf (all NaN): index 0, as main.c's loop leaves it */
		const int tok = bi == 0x7fffffff ? 0 : bi;
		btok[blockIdx.x] = tok;
		if (tokens)
			tokens[(size_t)blockIdx.x * tstride + st->step] = tok;
	}
}

/* ---------------------------------------------------------------------- */
/* k_lm_embed: the step token's row of token_embd in any block type         */
/* ---------------------------------------------------------------------- */

/*
 * out[K] = the dequantized row of the step's token (tensor_pick_rows,
 * tensor.c:263-294, through dequant_row, quant.c:420-575), element by
 * element with the reference's roundings: Q8_0 d * q, Q4_0 d * (n - 8),
 * Q4_K fl(fl(d * sc) * q) - fl(dmin * m) with the 6-bit scale and min of
 * the element's 32-value group (get_scale_min_k4, quant.h:60-69), Q6_K
 * fl(fl(d * sc) * q) with the signed scale of its 16 values.
 */
template <int WT>
__global__ __launch_bounds__(LM_NT) void k_lm_embed(const uint8_t *__restrict__ wte, int K,
						    const LmState *__restrict__ st,
						    const int *__restrict__ prompt,
						    float *__restrict__ out)
{
	const size_t rb = WT == 1   ? (size_t)(K / 32) * 34
			  : WT == 2 ? (size_t)(K / 32) * 18
			  : WT == 3 ? (size_t)(K / 256) * 144
				    : (size_t)(K / 256) * 210;
	const uint8_t *row = wte + (size_t)step_token(st, prompt) * rb;
	for (int e = threadIdx.x; e < K; e += LM_NT) {
		float v;
		if constexpr (WT == 1 || WT == 2) {
			const float4 q4 = dequant4<WT>(row, e / 4);
			v = (e & 3) == 0 ? q4.x : (e & 3) == 1 ? q4.y : (e & 3) == 2 ? q4.z : q4.w;
		} else if constexpr (WT == 3) {
			const uint8_t *b = row + (size_t)(e / 256) * 144;
			const int r = e % 256, j = r / 64, hi = (r % 64) / 32, g = r % 32;
			const int sb = 2 * j + hi; /* the 32-value group */
			const uint8_t *sc = b + 4;
			int sv, mv;
			if (sb < 4) {
				sv = sc[sb] & 63;
				mv = sc[sb + 4] & 63;
			} else {
				sv = (sc[sb + 4] & 0xF) | ((sc[sb - 4] >> 6) << 4);
				mv = (sc[sb + 4] >> 4) | ((sc[sb] >> 6) << 4);
			}
			const float d = f16_bits_to_f32((u32)b[0] | ((u32)b[1] << 8));
			const float dmin = f16_bits_to_f32((u32)b[2] | ((u32)b[3] << 8));
			const int qb = b[16 + 32 * j + g];
			const int q = hi ? qb >> 4 : qb & 0xF;
			const float ds = d * (float)sv, dm = dmin * (float)mv;
			const float t = ds * (float)q;
			v = t - dm;
		} else {
			const uint8_t *b = row + (size_t)(e / 256) * 210;
			const int r = e % 256, chunk = r / 128, rr = r % 128, quad = rr / 32,
				  l = rr % 32;
			const uint8_t *ql = b + 64 * chunk, *qh = b + 128 + 32 * chunk;
			const int lo = quad & 1 ? ql[l + 32] : ql[l];
			const int q = ((quad < 2 ? lo & 0xF : lo >> 4) | (((qh[l] >> (2 * quad)) & 3) << 4)) -
				      32;
			const int is = chunk * 8 + l / 16 + 2 * quad;
			const float d = f16_bits_to_f32((u32)b[208] | ((u32)b[209] << 8));
			const float ds = d * (float)(int8_t)b[192 + is];
			v = ds * (float)q;
		}
		out[e] = v;
	}
}

/* ---------------------------------------------------------------------- */
/* prefill: a prompt of T rows in one forward                              */
/* ---------------------------------------------------------------------- */

/*
 * k_lm_pf_qk: row t of sequence z (grid T x S) of a prompt's stacked q/k/v
 * product: the full-vector RMSNorms of q and k (OLMoE, olmoe.c:454-458),
 * RoPE at position pos0 + t on consecutive pairs of every head (rope_apply,
 * nn.c:192-219; the position is not clamped, as olmoe_prefill passes it,
 * olmoe.c:504-508), q into qo[z * T + t], k and v into the cache rows
 * size + t of every kv head (olmoe.c:276-289, llama.c:268-281).  The same
 * arithmetic as k_lm_attn's one row.
 */
__global__ __launch_bounds__(LM_NT) void k_lm_pf_qk(const float *__restrict__ qkv,
						    const float *__restrict__ q_norm,
						    const float *__restrict__ k_norm,
						    const float *__restrict__ freq,
						    float *__restrict__ kc, float *__restrict__ vc,
						    float *__restrict__ qo, int H, int KH, int C,
						    int size, int pos0, int T, size_t cstride)
{
	constexpr int HL = LM_HLEN;
	__shared__ float cs[HL / 2], sn[HL / 2];
	__shared__ float red[LM_NT / WAVE];
	const int t = blockIdx.x, z = blockIdx.y, EQ = H * HL, EK = KH * HL;
	const size_t r = (size_t)z * T + t;
	const float *q = qkv + r * (size_t)(EQ + 2 * EK), *k = q + EQ, *v = k + EK;
	kc += (size_t)z * cstride;
	vc += (size_t)z * cstride;
	float *qd = qo + r * (size_t)EQ;
	if (threadIdx.x < HL / 2) {
		const float ang = (float)(pos0 + t) * freq[threadIdx.x];
		cs[threadIdx.x] = cosf(ang);
		sn[threadIdx.x] = sinf(ang);
	}
	float rq = 1.0f, rk = 1.0f;
	if (q_norm) {
		float s1 = 0.0f, s2 = 0.0f;
		for (int i = threadIdx.x; i < EQ; i += LM_NT) {
			const float x = q[i] * q[i];
			s1 = s1 + x;
		}
		for (int i = threadIdx.x; i < EK; i += LM_NT) {
			const float x = k[i] * k[i];
			s2 = s2 + x;
		}
		rq = sqrtf(block_sum(s1, red) / (float)EQ + 1e-5f);
		rk = sqrtf(block_sum(s2, red) / (float)EK + 1e-5f);
	}
	__syncthreads();
	/* pair i of head h: item (h, i) of q's EQ / 2, then k's EK / 2 */
	for (int it = threadIdx.x; it < (EQ + EK) / 2; it += LM_NT) {
		const bool isq = it < EQ / 2;
		const int e = 2 * (isq ? it : it - EQ / 2), i = (e % HL) / 2;
		const float *src = isq ? q : k;
		const float *w = isq ? q_norm : k_norm;
		const float rr = isq ? rq : rk;
		float x0 = src[e], x1 = src[e + 1];
		if (q_norm) {
			x0 = (x0 / rr) * w[e];
			x1 = (x1 / rr) * w[e + 1];
		}
		const float co = cs[i], si = sn[i];
		const float y0 = __builtin_fmaf(x0, co, -(x1 * si));
		const float y1 = __builtin_fmaf(x0, si, x1 * co);
		if (isq) {
			qd[e] = y0;
			qd[e + 1] = y1;
		} else {
			const int kh = e / HL, d = e % HL;
			float *kr = kc + ((size_t)kh * C + size + t) * HL + d;
			kr[0] = y0;
			kr[1] = y1;
		}
	}
	for (int i = threadIdx.x; i < EK; i += LM_NT) {
		const int kh = i / HL, d = i % HL;
		vc[((size_t)kh * C + size + t) * HL + d] = v[i];
	}
}

#define PF_QB 64 /* query rows of a prefill attention workgroup */
#define PF_KB 64 /* cache rows per step of its key loop */

/*
 * k_lm_pf_attn: query head h of rows q0 .. q0 + PF_QB - 1 of sequence z
 * (grid H x ceil(T / PF_QB) x S) over the cache rows the causal mask (and
 * Mixtral's sliding window) leave it: query row t (absolute size + t) sees
 * rows j <= size + t, and with a window only size + t - j < window
 * (olmoe.c:309-320 with -1e4 for masked scores, whose exp is 0 as -inf's;
 * flash_attention's masks, nn.c:597-603).  Scores q . k / scale (OLMoE) or
 * * scale (Mixtral); the softmax runs online over blocks of PF_KB rows
 * (each block's maximum, the running sum rescaled), as flash_attention
 * does (nn.c:570-641), with a fully masked prefix taken as weight 0 rather
 * than exp(-inf - -inf).  Thread (row qi = tid / 4, quarter u = tid % 4)
 * holds dims 32u .. 32u + 31 of the row's q and of its output; the four
 * quarters' partial dots meet in two lane shuffles.
 */
__global__ __launch_bounds__(LM_NT) void k_lm_pf_attn(const float *__restrict__ qo,
						      const float *__restrict__ kc,
						      const float *__restrict__ vc,
						      float *__restrict__ out, int H, int KH, int C,
						      int size, int T, int window, float scale,
						      int scale_mul, size_t cstride)
{
	constexpr int HL = LM_HLEN, RS = HL + 4, SS = PF_KB + 1;
	static_assert(LM_NT == 4 * PF_QB, "four threads per query row");
	__shared__ __attribute__((aligned(16))) float sk[PF_KB * RS], sv[PF_KB * RS];
	/* a block's scores of each query row (kept in registers, unrolled, the
	 * 64 scores and their operands spilled ~6.5 KB a lane to scratch) */
	__shared__ float ssc[PF_QB * SS];
	const int h = blockIdx.x, q0 = blockIdx.y * PF_QB, z = blockIdx.z;
	const int EQ = H * HL, kh = h / (H / KH);
	const int tid = threadIdx.x, qi = tid / 4, u = tid % 4;
	const int t = q0 + qi;
	const bool live = t < T;
	kc += (size_t)z * cstride + (size_t)kh * C * HL;
	vc += (size_t)z * cstride + (size_t)kh * C * HL;
	float qv[32], o[32];
	{
		const float4 *q4 = (const float4 *)(qo + ((size_t)z * T + (live ? t : 0)) * EQ +
						    (size_t)h * HL + 32 * u);
#pragma unroll
		for (int i = 0; i < 8; i++) {
			const float4 v = q4[i];
			qv[4 * i] = v.x;
			qv[4 * i + 1] = v.y;
			qv[4 * i + 2] = v.z;
			qv[4 * i + 3] = v.w;
		}
	}
#pragma unroll
	for (int i = 0; i < 32; i++)
		o[i] = 0.0f;
	const int qa = size + t; /* this row's absolute position in the cache */
	const int tlast = min(q0 + PF_QB, T) - 1;
	const int jhi = size + tlast + 1; /* rows the block's last query sees */
	const int jlo = window > 0 ? max(0, size + q0 - window + 1) : 0;
	float m = -INFINITY, l = 0.0f;
	for (int j0 = jlo; j0 < jhi; j0 += PF_KB) {
		__syncthreads(); /* the previous block's readers are done */
		for (int e = tid; e < PF_KB * HL / 4; e += LM_NT) {
			const int jj = e / (HL / 4), c4 = e % (HL / 4);
			float4 kv = {0.0f, 0.0f, 0.0f, 0.0f}, vv = kv;
			if (j0 + jj < jhi) {
				kv = ((const float4 *)(kc + (size_t)(j0 + jj) * HL))[c4];
				vv = ((const float4 *)(vc + (size_t)(j0 + jj) * HL))[c4];
			}
			*(float4 *)(sk + jj * RS + 4 * c4) = kv;
			*(float4 *)(sv + jj * RS + 4 * c4) = vv;
		}
		__syncthreads();
		float *sc = ssc + qi * SS;
#pragma unroll 2
		for (int jj = 0; jj < PF_KB; jj++) {
			const float4 *k4 = (const float4 *)(sk + jj * RS + 32 * u);
			float a = 0.0f;
#pragma unroll
			for (int i = 0; i < 8; i++) {
				const float4 kv = k4[i];
				a = __builtin_fmaf(qv[4 * i], kv.x, a);
				a = __builtin_fmaf(qv[4 * i + 1], kv.y, a);
				a = __builtin_fmaf(qv[4 * i + 2], kv.z, a);
				a = __builtin_fmaf(qv[4 * i + 3], kv.w, a);
			}
			a += __shfl_xor(a, 1, WAVE);
			a += __shfl_xor(a, 2, WAVE);
			const int j = j0 + jj;
			const bool keep = j <= qa && (window <= 0 || qa - j < window);
			if (u == 0)
				sc[jj] = keep ? (scale_mul ? a * scale : a / scale) : -INFINITY;
		}
		__syncthreads(); /* the row's scores, from its quarter 0 */
		float mb = -INFINITY;
#pragma unroll 8
		for (int jj = 0; jj < PF_KB; jj++)
			mb = fmaxf(mb, sc[jj]);
		const float mn = fmaxf(m, mb);
		if (mn == -INFINITY)
			continue; /* nothing of this row so far */
		const float corr = m == -INFINITY ? 0.0f : moe_expf(m - mn);
		l = l * corr;
#pragma unroll
		for (int i = 0; i < 32; i++)
			o[i] = o[i] * corr;
#pragma unroll 2
		for (int jj = 0; jj < PF_KB; jj++) {
			const float sj = sc[jj];
			const float pj = sj == -INFINITY ? 0.0f : moe_expf(sj - mn);
			l = l + pj;
			const float4 *v4 = (const float4 *)(sv + jj * RS + 32 * u);
#pragma unroll
			for (int i = 0; i < 8; i++) {
				const float4 vv = v4[i];
				o[4 * i] = __builtin_fmaf(pj, vv.x, o[4 * i]);
				o[4 * i + 1] = __builtin_fmaf(pj, vv.y, o[4 * i + 1]);
				o[4 * i + 2] = __builtin_fmaf(pj, vv.z, o[4 * i + 2]);
				o[4 * i + 3] = __builtin_fmaf(pj, vv.w, o[4 * i + 3]);
			}
		}
		m = mn;
	}
	if (live) {
		float4 *o4 = (float4 *)(out + ((size_t)z * T + t) * EQ + (size_t)h * HL + 32 * u);
#pragma unroll
		for (int i = 0; i < 8; i++)
			o4[i] = float4{o[4 * i] / l, o[4 * i + 1] / l, o[4 * i + 2] / l, o[4 * i + 3] / l};
	}
}

/* ---------------------------------------------------------------------- */
/* launchers                                                              */
/* ---------------------------------------------------------------------- */

static size_t tok_lds(int K)
{
	return (size_t)(K / MOE_SEG_COLS) * SEG_STRIDE * sizeof(float);
}

/* the instance of kind k (0 qkv, 1 oproj, 2 head) for (wtype, K) */
static const void *lm_kernel(int kind, int wtype, int K)
{
	const int C = moe_lanes_per_row((size_t)K);
#define LMK(WTT, CC)                                                                    \
	if (wtype == WTT && C == CC)                                                    \
		return kind == 0 ? (const void *)k_lm_qkv<WTT, CC>                       \
		       : kind == 1 ? (const void *)k_lm_oproj<WTT, CC>                   \
				   : (const void *)k_lm_head<WTT, CC>;
	LMK(1, 4) LMK(1, 8) LMK(1, 16) LMK(1, 32) LMK(1, 64)
	LMK(2, 4) LMK(2, 8) LMK(2, 16) LMK(2, 32) LMK(2, 64)
#undef LMK
	return nullptr;
}

/* compute units of the current device (256 if the query fails), cached
 * per device: the attention launch asks at every step, also under capture */
static int lm_cus()
{
	static int cus[64];
	int dev = 0, ncu = 0;
	if (hipGetDevice(&dev) != hipSuccess)
		return 256;
	if (dev >= 0 && dev < 64 && cus[dev] > 0)
		return cus[dev];
	if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
	    ncu < 1)
		return 256;
	if (dev >= 0 && dev < 64)
		__atomic_store_n(&cus[dev], ncu, __ATOMIC_RELAXED);
	return ncu;
}

extern "C" int lm_gemv_grid(int kind, int wtype, int K, int N)
{
	const void *fn = lm_kernel(kind, wtype, K);
	int dev = 0, ncu = 0, per = 0;
	if (!fn || hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
	    hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, LM_NT, tok_lds(K)) != hipSuccess ||
	    per < 1)
		return 0;
	const int C = moe_lanes_per_row((size_t)K);
	const int ngroups = (N + QG_WAVES * (WAVE / C) - 1) / (QG_WAVES * (WAVE / C));
	return min(ngroups, per * ncu);
}

extern "C" int lm_launch_qkv(int wtype, const uint8_t *W, int N, int K, const float *a,
			     const float *b, const float *w, float *h_out, const uint8_t *wte,
			     const LmState *st, const int *prompt, float *out, int grid,
			     void *stream)
{
	const void *fn = lm_kernel(0, wtype, K);
	if (!fn || grid < 1)
		return (int)hipErrorInvalidValue;
	size_t rb = (size_t)(K / MOE_QK) * (wtype == 1 ? 34 : 18);
	void *args[] = {&W, &rb, &N, &K, &a, &b, &w, &h_out, &wte, &st, &prompt, &out};
	return (int)hipLaunchKernel(fn, dim3(grid), dim3(LM_NT), args, tok_lds(K),
				    (hipStream_t)stream);
}

extern "C" int lm_launch_oproj(int wtype, const uint8_t *W, int N, int K, const float *x,
			       const float *add, float *out, uint64_t *rows_t, const float *w,
			       float *x_out, LmState *st, int layer, int grid, void *stream)
{
	const void *fn = lm_kernel(1, wtype, K);
	if (!fn || grid < 1 || grid > LM_MAX_HEAD_WG || N > (int)(tok_lds(K) / sizeof(float)))
		return (int)hipErrorInvalidValue;
	size_t rb = (size_t)(K / MOE_QK) * (wtype == 1 ? 34 : 18);
	void *args[] = {&W, &rb, &N, &K, &x, &add, &out, &rows_t, &w, &x_out, &st, &layer};
	return (int)hipLaunchKernel(fn, dim3(grid), dim3(LM_NT), args, tok_lds(K),
				    (hipStream_t)stream);
}

extern "C" int lm_launch_head(int wtype, const uint8_t *W, int N, int K, const float *a,
			      const float *b, const float *w, float *out, uint64_t *best,
			      LmState *st, int *tokens, int grid, void *stream)
{
	const void *fn = lm_kernel(2, wtype, K);
	if (!fn || grid < 1 || grid > LM_MAX_HEAD_WG)
		return (int)hipErrorInvalidValue;
	size_t rb = (size_t)(K / MOE_QK) * (wtype == 1 ? 34 : 18);
	void *args[] = {&W, &rb, &N, &K, &a, &b, &w, &out, &best, &st, &tokens};
	return (int)hipLaunchKernel(fn, dim3(grid), dim3(LM_NT), args, tok_lds(K),
				    (hipStream_t)stream);
}

extern "C" int lm_attn_chunks(int C, int window)
{
	const int span = window > 0 && window < C ? window : C;
	return (span + LM_CHUNK - 1) / LM_CHUNK;
}

/* 2: the attention grid of kh kv heads, nact chunks and nseq sequences is
 * resident at once and chunk 0 merges; 1: the last chunk to count in
 * merges (the current device) */
extern "C" int lm_attn_merge_form(int KH, int nact, int nseq)
{
	return (size_t)KH * nact * nseq <= 3 * (size_t)lm_cus() ? 2 : 1;
}

extern "C" int lm_launch_attn(const float *qkv, const float *q_norm, const float *k_norm,
			      const float *freq, LmState *st, float *kc, float *vc,
			      uint64_t *part, uint32_t *cnt, float *out, int H, int KH, int C,
			      int window, float scale, int scale_mul, int layer, int nact,
			      int nseq, size_t cstride, void *stream)
{
	const int nch = lm_attn_chunks(C, window);
	if (KH < 1 || H % KH || nch > LM_MAX_CHUNKS || nact < 1 || nact > nch || layer < 0 ||
	    layer >= LM_HEAD_SLOT || nseq < 1 || nseq > 65535)
		return (int)hipErrorInvalidValue;
	const dim3 grid(KH, nact, nseq);
	hipStream_t s = (hipStream_t)stream;
	/* all of a chunk's rows loaded early while the grid fits 3 workgroups
	 * per CU at once; larger grids load k early and v before its use (at
	 * a register count that keeps more workgroups resident) */
	const bool pf = lm_attn_merge_form(KH, nact, nseq) == 2;
#define ATTN(GG)                                                                               \
	do {                                                                                   \
		if (pf)                                                                        \
			hipLaunchKernelGGL((k_lm_attn<GG, 2>), grid, dim3(LM_NT), 0, s, qkv,      \
					   q_norm, k_norm, freq, st, kc, vc, part, cnt, out, H, KH,   \
					   C, window, scale, scale_mul, layer, nch, cstride);         \
		else                                                                           \
			hipLaunchKernelGGL((k_lm_attn<GG, 1>), grid, dim3(LM_NT), 0, s, qkv,      \
					   q_norm, k_norm, freq, st, kc, vc, part, cnt, out, H, KH,   \
					   C, window, scale, scale_mul, layer, nch, cstride);         \
	} while (0)
	switch (H / KH) {
	case 1: ATTN(1); break;
	case 2: ATTN(2); break;
	case 4: ATTN(4); break;
	case 8: ATTN(8); break;
	default: return (int)hipErrorInvalidValue;
	}
#undef ATTN
	return (int)hipGetLastError();
}

extern "C" int lm_launch_norm_rows(int wtype, int nseq, int E, const float *a, const float *b,
				   const float *w, float *h_out, float *x_out, const uint8_t *wte,
				   const LmState *st, const int *prompt, const int *btok,
				   void *stream)
{
	if (nseq < 1 || E % MOE_SEG_COLS || (!a && (!wte || !prompt || !btok)))
		return (int)hipErrorInvalidValue;
	const size_t lds = tok_lds(E);
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		hipLaunchKernelGGL(k_lm_norm_rows<1>, dim3(nseq), dim3(LM_NT), lds, s, E, a, b, w,
				   h_out, x_out, wte, st, prompt, btok);
	else if (wtype == 2)
		hipLaunchKernelGGL(k_lm_norm_rows<2>, dim3(nseq), dim3(LM_NT), lds, s, E, a, b, w,
				   h_out, x_out, wte, st, prompt, btok);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int lm_launch_norm_parts(int nseq, int E, const float *part, int KS, size_t TN,
				    const float *add, const float *w, float *h_out, float *x_out,
				    void *stream)
{
	if (nseq < 1 || E % 4 || KS < 1 || TN < (size_t)nseq * E || !part || !add || !w ||
	    !h_out || !x_out)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_lm_norm_parts, dim3(nseq), dim3(LM_NT), (size_t)E * sizeof(float),
			   (hipStream_t)stream, E, part, KS, TN, add, w, h_out, x_out);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_pick_rows(const float *logits, int nseq, int V, const LmState *st,
				   int *btok, int *tokens, int tstride, void *stream)
{
	if (nseq < 1 || V < 1)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_lm_pick_rows, dim3(nseq), dim3(PK_NT), 0, (hipStream_t)stream, logits,
			   V, st, btok, tokens, tstride);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_step_end(LmState *st, void *stream)
{
	hipLaunchKernelGGL(k_lm_step_end, dim3(1), dim3(64), 0, (hipStream_t)stream, st);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_copy_rows(const float *src, float *dst, size_t slab, size_t n,
				   size_t slabs, void *stream)
{
	if (slabs == 0 || n == 0)
		return 0;
	hipLaunchKernelGGL(k_lm_copy_rows, dim3(64, (unsigned)slabs), dim3(256), 0,
			   (hipStream_t)stream, src, dst, slab, n);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_pf_qk(const float *qkv, const float *q_norm, const float *k_norm,
			       const float *freq, float *kc, float *vc, float *qo, int H, int KH,
			       int C, int size, int pos0, int T, int nseq, size_t cstride,
			       void *stream)
{
	if (T < 1 || nseq < 1 || nseq > 65535 || KH < 1 || H % KH || size < 0 || size + T > C ||
	    (!q_norm) != (!k_norm))
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_lm_pf_qk, dim3(T, nseq), dim3(LM_NT), 0, (hipStream_t)stream, qkv,
			   q_norm, k_norm, freq, kc, vc, qo, H, KH, C, size, pos0, T, cstride);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_pf_attn(const float *qo, const float *kc, const float *vc, float *out,
				 int H, int KH, int C, int size, int T, int window, float scale,
				 int scale_mul, int nseq, size_t cstride, void *stream)
{
	if (T < 1 || nseq < 1 || nseq > 65535 || KH < 1 || H % KH || size < 0 || size + T > C ||
	    (T + PF_QB - 1) / PF_QB > 65535)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(k_lm_pf_attn, dim3(H, (T + PF_QB - 1) / PF_QB, nseq), dim3(LM_NT), 0,
			   (hipStream_t)stream, qo, kc, vc, out, H, KH, C, size, T, window, scale,
			   scale_mul, cstride);
	return (int)hipGetLastError();
}

extern "C" int lm_launch_embed(int wtype, const uint8_t *wte, int K, const LmState *st,
			       const int *prompt, float *out, void *stream)
{
	hipStream_t s = (hipStream_t)stream;
	if ((wtype == 1 || wtype == 2) && K % 32 == 0) {
		if (wtype == 1)
			hipLaunchKernelGGL(k_lm_embed<1>, dim3(1), dim3(LM_NT), 0, s, wte, K, st, prompt, out);
		else
			hipLaunchKernelGGL(k_lm_embed<2>, dim3(1), dim3(LM_NT), 0, s, wte, K, st, prompt, out);
	} else if ((wtype == 3 || wtype == 5) && K % 256 == 0) {
		if (wtype == 3)
			hipLaunchKernelGGL(k_lm_embed<3>, dim3(1), dim3(LM_NT), 0, s, wte, K, st, prompt, out);
		else
			hipLaunchKernelGGL(k_lm_embed<5>, dim3(1), dim3(LM_NT), 0, s, wte, K, st, prompt, out);
	} else {
		return (int)hipErrorInvalidValue;
	}
	return (int)hipGetLastError();
}
