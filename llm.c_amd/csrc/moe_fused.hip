/*
 * Decode-sized MoE FFN layer (T*K <= 64) in two launches.
 *
 * k_route_decode (one workgroup per router item, no waiting):
 *   each active wave owns one expert j and computes logits[t][j] for every
 *   token with the 8-lane FMA chains of dot_f32_f32 (matmul.c:91-105), fed
 *   from LDS-transposed copies of the router row and the token; the last
 *   router item to finish runs softmax + top-k (+ renorm) for every token
 *   (nn.c:221-308, llama.c:422-427) and writes ids/w.
 *
 * k_experts (persistent; the rest of moe_ffn, olmoe.c:364-406):
 *   gate/up items  16 rows of gate and up of the expert in slot p:
 *                  h[p][row] = silu(gate.x) * (up.x)          (nn.c:460-478)
 *   down items     32 rows of down over one K-chunk of h[p]  (nn.c:490-492);
 *                  the last item to finish a (token, row block) combines the
 *                  slots in order: out += y / (1/w)  (olmoe.c:401-403).
 *
 * Items are claimed from NQ ticket queues (workgroup b uses queue b % NQ;
 * queue q holds items q, q+NQ, ... in order), gate/up items before down
 * items.  A down item waits only for its slot's gate/up items, which precede
 * it in every queue; an item claimed from a queue belongs to a running
 * workgroup and gate/up items never wait, so every wait ends: no grid
 * barrier and no co-residency assumption.  Waits are bounded anyway; one
 * that runs out sets an error word instead of hanging.  The last workgroup to
 * exit zeroes the counters for the next launch.
 *
 * Data another workgroup produced in the same launch (logits, h, partial y)
 * is written with device-coherent stores (agent-scope relaxed atomics: `sc1`
 * on gfx950, written through the per-XCD L2) and read with device-coherent
 * loads.  A producer waits for its stores to complete (s_waitcnt) before the
 * barrier and the counter increment, so a consumer that has seen the counter
 * reads the data.  Agent-scope release/acquire fences are avoided: on gfx950
 * they write back / invalidate a whole XCD L2 (buffer_wbl2 / buffer_inv).
 * Every counter sits on its own 256-byte line, and pollers back off.
 */
#include "moe_device.h"

#define GU_ROWS 16
#define DN_ROWS 32
#define NTHREADS 256
#define NQ 8

/* counter lines: word index = line * SYNC_LINE */
#define SYNC_LINE 64
enum {
	L_ROUTED = 0,
	L_EXIT = 1,
	L_ERR = MOE_SYNC_ERR_WORD / SYNC_LINE,
	L_TICKET = 8,        /* NQ lines */
	L_GU = 8 + NQ,       /* P lines, then T * (E / DN_ROWS) combine lines */
};
#define W(line) ((line) * SYNC_LINE)

struct FusedArgs {
	const float *x;
	const float *router;
	const float *bias;
	const uint8_t *gate, *up, *down;
	size_t gu_stride, dn_stride;
	float *logits;
	u32 *ids;
	float *w;
	float *h;
	float *ypart;
	float *out;
	u32 *sync;
	int T, E, EI, NE, K, renorm, kch;
	int n_rt, n_gu, n_dn;
	int rt_experts;
	int nlines;
};

#define SPIN_LIMIT (1 << 20)

/* device-coherent data accesses (global_{load,store} ... sc1) */
__device__ static inline void st_dev(float *p, float v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline float ld_dev(const float *p)
{
	return __hip_atomic_load((float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline float2 ld_dev2(const float *p)
{
	uint64_t v = __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
	return __builtin_bit_cast(float2, v);
}
__device__ static inline u32 ld_relaxed(u32 *p)
{
	return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline u32 fetch_add(u32 *p)
{
	return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* thread 0 polls until *p >= target with a growing back-off; the barrier
 * then holds every thread. */
__device__ static inline void wait_geq(u32 *p, u32 target, u32 *err)
{
	if (threadIdx.x == 0) {
		int i = 0, step = 0;
		while (ld_relaxed(p) < target) {
			switch (step) {
			case 0: __builtin_amdgcn_s_sleep(1); break;
			case 1: __builtin_amdgcn_s_sleep(2); break;
			case 2: __builtin_amdgcn_s_sleep(4); break;
			case 3: __builtin_amdgcn_s_sleep(8); break;
			default: __builtin_amdgcn_s_sleep(16); break;
			}
			step += step < 4;
			if (++i >= SPIN_LIMIT) {
				__hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
				break;
			}
		}
	}
	__syncthreads();
}

/* every thread's device-coherent stores complete, then thread 0 bumps the
 * counter; returns the counter's previous value to every thread */
__device__ static inline u32 signal_add(u32 *p)
{
	__builtin_amdgcn_s_waitcnt(0);
	__syncthreads();
	__shared__ u32 s_old;
	if (threadIdx.x == 0)
		s_old = fetch_add(p);
	__syncthreads();
	return s_old;
}

/* the same without waiting for the counter's reply */
__device__ static inline void signal_post(u32 *p)
{
	__builtin_amdgcn_s_waitcnt(0);
	__syncthreads();
	if (threadIdx.x == 0)
		__hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* stage_padded for data another workgroup produced in this launch */
__device__ static inline void stage_padded_dev(float *s, const float *g, int n, int tid)
{
	for (int i = tid; i < n / 2; i += NTHREADS) {
		float2 v = ld_dev2(g + 2 * i);
		int k = 2 * i;
		*(float2 *)(s + (k >> 6) * SEG_STRIDE + (k & 63)) = v;
	}
}

/* ---------------------------------------------------------------------- */
/* routing                                                                */
/* ---------------------------------------------------------------------- */

/* copy n floats, element k -> dst[(k & 7) * RS + (k >> 3)] */
__device__ static inline void stage_transposed(float *dst, const float *src, int n, int RS,
					       int tid, int nthreads)
{
	const float4 *s4 = (const float4 *)src;
	for (int i = tid; i < n / 4; i += nthreads) {
		float4 v = s4[i];
		int k = 4 * i;
		dst[((k + 0) & 7) * RS + ((k + 0) >> 3)] = v.x;
		dst[((k + 1) & 7) * RS + ((k + 1) >> 3)] = v.y;
		dst[((k + 2) & 7) * RS + ((k + 2) >> 3)] = v.z;
		dst[((k + 3) & 7) * RS + ((k + 3) >> 3)] = v.w;
	}
}

__global__ __launch_bounds__(NTHREADS) void k_route_decode(FusedArgs a)
{
	extern __shared__ float lds[];
	const int E = a.E, E8 = E / 8, RS = E8 + 4;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	float *sx = lds;          /* [8][RS] token, transposed */
	float *sw = lds + 8 * RS; /* [rt_experts][8][RS] router rows */
	const int j = blockIdx.x * a.rt_experts + wave;
	const bool active = wave < a.rt_experts && j < a.NE;

	if (active)
		stage_transposed(sw + wave * 8 * RS, a.router + (size_t)j * E, E, RS, lane, WAVE);
	for (int t = 0; t < a.T; t++) {
		stage_transposed(sx, a.x + (size_t)t * E, E, RS, tid, NTHREADS);
		__syncthreads();
		if (active) {
			/* lane l < 8 replays AVX2 lane l: elements l, l+8, ... in order */
			const int l = lane & 7;
			const float4 *xr = (const float4 *)(sx + l * RS);
			const float4 *wr = (const float4 *)(sw + (wave * 8 + l) * RS);
			float acc = 0.0f;
#pragma unroll 16
			for (int i = 0; i < E8 / 4; i++) {
				float4 xv = xr[i], wv = wr[i];
				acc = __builtin_fmaf(xv.x, wv.x, acc);
				acc = __builtin_fmaf(xv.y, wv.y, acc);
				acc = __builtin_fmaf(xv.z, wv.z, acc);
				acc = __builtin_fmaf(xv.w, wv.w, acc);
			}
			acc = acc + __shfl_xor(acc, 4, 8);
			acc = acc + __shfl_xor(acc, 2, 8);
			acc = acc + __shfl_xor(acc, 1, 8);
			if (lane == 0)
				st_dev(&a.logits[(size_t)t * a.NE + j],
				       (a.bias ? a.bias[j] : 0.0f) + acc);
		}
		__syncthreads();
	}

	u32 done = signal_add(&a.sync[W(L_ROUTED)]);
	if (done != (u32)a.n_rt - 1)
		return;
	/* last router item: softmax/top-k per token, one wave per token, on a
	 * device-coherent copy of the logits in LDS */
	float *sp = lds + wave * (2 * MOE_MAX_NE + 4 * MOE_MAX_TOPK);
	float *slg = sp + MOE_MAX_NE;
	u32 *sid = (u32 *)(slg + MOE_MAX_NE);
	float *swt = (float *)(sid + MOE_MAX_TOPK);
	for (int t = wave; t < a.T; t += NTHREADS / WAVE) {
		for (int i = lane; i < a.NE; i += WAVE)
			slg[i] = ld_dev(&a.logits[(size_t)t * a.NE + i]);
		WAVE_SYNC();
		wave_softmax_topk(slg, NULL, a.ids + (size_t)t * a.K, a.w + (size_t)t * a.K, a.NE,
				  a.K, a.renorm, sp, sid, swt, lane);
	}
	if (tid == 0) /* every router item has counted: ready for the next launch */
		__hip_atomic_store(&a.sync[W(L_ROUTED)], 0u, __ATOMIC_RELAXED,
				   __HIP_MEMORY_SCOPE_AGENT);
}

/* ---------------------------------------------------------------------- */
/* experts                                                                */
/* ---------------------------------------------------------------------- */

template <int WT, int CG>
__device__ static void gateup_item(const FusedArgs &a, int g, float *sact, int &staged_tok)
{
	constexpr int RPS = WAVE / CG, RW = GU_ROWS / 4;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int tiles = a.EI / GU_ROWS;
	const int p = g / tiles, row0 = (g % tiles) * GU_ROWS + wave * RW;
	const int t = p / a.K;
	const int e = (int)a.ids[p];

	if (staged_tok != t) { /* the item loop's barrier retired earlier readers */
		stage_padded(sact, a.x + (size_t)t * a.E, a.E, tid, NTHREADS);
		__syncthreads();
		staged_tok = t;
	}
	const int seg = lane % CG, sub = lane / CG;
	float xr[64];
	lds_x64(sact, seg, xr);

	const size_t rb = (size_t)(a.E / MOE_QK) * (qseg<WT>::BYTES / 2);
	const uint8_t *G = a.gate + (size_t)e * a.gu_stride + (size_t)seg * qseg<WT>::BYTES;
	const uint8_t *U = a.up + (size_t)e * a.gu_stride + (size_t)seg * qseg<WT>::BYTES;
#pragma unroll
	for (int r = 0; r < RW; r += RPS) {
		const int row = row0 + r + sub;
		float gv = qseg<WT>::dot(G + (size_t)row * rb, xr);
		float uv = qseg<WT>::dot(U + (size_t)row * rb, xr);
		gv = group_sum<CG>(gv);
		uv = group_sum<CG>(uv);
		if (seg == 0)
			st_dev(&a.h[(size_t)p * a.EI + row], (gv / (1.0f + moe_expf(-gv))) * uv);
	}
	signal_post(&a.sync[W(L_GU + p)]);
}

template <int WT, int CD>
__device__ static void down_item(const FusedArgs &a, int d, float *sh, uint64_t &gu_seen)
{
	constexpr int RPS = WAVE / CD, RW = DN_ROWS / 4;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int nrb = a.E / DN_ROWS;
	const int p = d / (a.kch * nrb), rem = d % (a.kch * nrb);
	const int kc = rem / nrb, rbk = rem % nrb;
	const int t = p / a.K;
	const int row0 = rbk * DN_ROWS + wave * RW;
	const int e = (int)a.ids[p];

	if (!(gu_seen >> p & 1)) { /* h[p] complete */
		wait_geq(&a.sync[W(L_GU + p)], (u32)(a.EI / GU_ROWS), &a.sync[W(L_ERR)]);
		gu_seen |= (uint64_t)1 << p;
	}
	stage_padded_dev(sh, a.h + (size_t)p * a.EI + (size_t)kc * CD * MOE_SEG_COLS,
			 CD * MOE_SEG_COLS, tid);
	__syncthreads();
	const int seg = lane % CD, sub = lane / CD;
	float xr[64];
	lds_x64(sh, seg, xr);

	const size_t rb = (size_t)(a.EI / MOE_QK) * (qseg<WT>::BYTES / 2);
	const uint8_t *D = a.down + (size_t)e * a.dn_stride +
			   (size_t)(kc * CD + seg) * qseg<WT>::BYTES;
#pragma unroll
	for (int r = 0; r < RW; r += RPS) {
		const int row = row0 + r + sub;
		float y = group_sum<CD>(qseg<WT>::dot(D + (size_t)row * rb, xr));
		if (seg == 0)
			st_dev(&a.ypart[((size_t)p * a.kch + kc) * a.E + row], y);
	}
	u32 old = signal_add(&a.sync[W(L_GU + a.T * a.K + t * nrb + rbk)]);
	if (old != (u32)(a.K * a.kch) - 1)
		return;
	/* last contribution to this (token, row block): combine in slot order */
	if (tid < DN_ROWS) {
		const int row = rbk * DN_ROWS + tid;
		float acc = 0.0f;
		for (int s = 0; s < a.K; s++) {
			const size_t ps = (size_t)t * a.K + s;
			float y = ld_dev(&a.ypart[ps * a.kch * a.E + row]);
			for (int c = 1; c < a.kch; c++)
				y += ld_dev(&a.ypart[(ps * a.kch + c) * a.E + row]);
			acc = acc + y / (1.0f / a.w[ps]);
		}
		a.out[(size_t)t * a.E + row] = acc;
	}
}

template <int WT, int CG, int CD>
__global__ __launch_bounds__(NTHREADS) void k_experts(FusedArgs a)
{
	extern __shared__ float lds[];
	__shared__ int s_ticket;
	const int tid = threadIdx.x;
	const int q = blockIdx.x % NQ;
	const int total = a.n_gu + a.n_dn;
	u32 *ticket = &a.sync[W(L_TICKET + q)];
	float *sact = lds;                                   /* x, padded */
	float *sh = lds + (a.E / MOE_SEG_COLS) * SEG_STRIDE; /* h chunk, padded */
	int staged_tok = -1;
	uint64_t gu_seen = 0;

	if (tid == 0)
		s_ticket = (int)fetch_add(ticket);
	__syncthreads();
	int item = q + NQ * s_ticket;
	while (item < total) {
		u32 nxt = 0;
		if (tid == 0)
			nxt = fetch_add(ticket);
		if (item < a.n_gu)
			gateup_item<WT, CG>(a, item, sact, staged_tok);
		else
			down_item<WT, CD>(a, item - a.n_gu, sh, gu_seen);
		__syncthreads();
		if (tid == 0)
			s_ticket = (int)nxt;
		__syncthreads();
		item = q + NQ * s_ticket;
	}

	/* the last workgroup out zeroes the counters for the next launch */
	__shared__ int s_last;
	if (tid == 0)
		s_last = fetch_add(&a.sync[W(L_EXIT)]) == gridDim.x - 1;
	__syncthreads();
	if (s_last)
		for (int i = tid; i < a.nlines; i += NTHREADS)
			if (i != L_ERR && i != L_ROUTED)
				__hip_atomic_store(&a.sync[W(i)], 0u, __ATOMIC_RELAXED,
						   __HIP_MEMORY_SCOPE_AGENT);
}

/* ---------------------------------------------------------------------- */

template <int WT, int CG, int CD>
static const void *experts_fn()
{
	return (const void *)k_experts<WT, CG, CD>;
}

static const void *pick_experts(int wtype, int CG, int CD)
{
#define F3(W_, G, D)                                  \
	if (wtype == W_ && CG == G && CD == D)        \
		return experts_fn<W_, G, D>();
#define FD(W_, G) F3(W_, G, 16) F3(W_, G, 32) F3(W_, G, 64)
	FD(1, 16) FD(1, 32) FD(1, 64) FD(2, 16) FD(2, 32) FD(2, 64)
#undef FD
#undef F3
	return NULL;
}

static int rt_experts_for(int E)
{
	return E <= 1024 ? 4 : (E <= 2048 ? 2 : 1);
}

static size_t route_lds_bytes(int E)
{
	size_t rt = (size_t)(rt_experts_for(E) + 1) * 8 * (E / 8 + 4) * sizeof(float);
	size_t tk = (size_t)4 * (2 * MOE_MAX_NE + 4 * MOE_MAX_TOPK) * sizeof(float);
	return rt > tk ? rt : tk;
}

static size_t experts_lds_bytes(int E, int EI)
{
	int CD = moe_lanes_per_row((size_t)EI);
	return (size_t)(E / MOE_SEG_COLS + CD) * SEG_STRIDE * sizeof(float);
}

extern "C" int moe_fused_supported(int wtype, size_t E, size_t EI, size_t T, size_t K)
{
	int CG = moe_lanes_per_row(E);
	if (moe_kchunks(E) != 1)
		return 0;
	int CD = moe_lanes_per_row(EI);
	if (T * K > MOE_FUSED_MAX_P || E % DN_ROWS || EI % GU_ROWS)
		return 0;
	return pick_experts(wtype, CG, CD) != NULL;
}

static size_t sync_lines(size_t T, size_t K, size_t E)
{
	return L_GU + T * K + T * (E / DN_ROWS);
}

extern "C" size_t moe_fused_sync_words(size_t T, size_t K, size_t E)
{
	return sync_lines(T, K, E) * SYNC_LINE;
}

extern "C" int moe_fused_grid(int wtype, size_t E, size_t EI)
{
	int CG = moe_lanes_per_row(E), CD = moe_lanes_per_row(EI);
	const void *fn = pick_experts(wtype, CG, CD);
	if (!fn)
		return 0;
	int dev = 0, ncu = 0, per = 0;
	if (hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		return 0;
	if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, NTHREADS,
							 experts_lds_bytes((int)E, (int)EI)) !=
		    hipSuccess ||
	    per < 1)
		per = 1;
	if (per > MOE_FUSED_WG_PER_CU)
		per = MOE_FUSED_WG_PER_CU;
	return ncu * per;
}

extern "C" int moe_launch_fused(int wtype, const float *x, const float *router,
				const float *bias, const uint8_t *gate, const uint8_t *up,
				const uint8_t *down, size_t gu_stride, size_t dn_stride,
				float *logits, uint32_t *ids, float *w, float *h, float *ypart,
				float *out, uint32_t *sync, int T, int E, int EI, int NE, int K,
				int renorm, int grid, void *stream)
{
	int CG = moe_lanes_per_row((size_t)E), CD = moe_lanes_per_row((size_t)EI);
	const void *fn = pick_experts(wtype, CG, CD);
	if (!fn || grid < NQ)
		return (int)hipErrorInvalidValue;
	FusedArgs a;
	a.x = x;
	a.router = router;
	a.bias = bias;
	a.gate = gate;
	a.up = up;
	a.down = down;
	a.gu_stride = gu_stride;
	a.dn_stride = dn_stride;
	a.logits = logits;
	a.ids = ids;
	a.w = w;
	a.h = h;
	a.ypart = ypart;
	a.out = out;
	a.sync = sync;
	a.T = T;
	a.E = E;
	a.EI = EI;
	a.NE = NE;
	a.K = K;
	a.renorm = renorm;
	a.kch = moe_kchunks((size_t)EI);
	a.rt_experts = rt_experts_for(E);
	a.n_rt = (NE + a.rt_experts - 1) / a.rt_experts;
	a.n_gu = T * K * (EI / GU_ROWS);
	a.n_dn = T * K * a.kch * (E / DN_ROWS);
	a.nlines = (int)sync_lines((size_t)T, (size_t)K, (size_t)E);
	int total = a.n_gu + a.n_dn;
	if (grid > total)
		grid = total < NQ ? NQ : total;
	void *args[] = {&a};
	hipError_t rc = hipLaunchKernel((const void *)k_route_decode, dim3(a.n_rt), dim3(NTHREADS),
					args, route_lds_bytes(E), (hipStream_t)stream);
	if (rc != hipSuccess)
		return (int)rc;
	rc = hipLaunchKernel(fn, dim3(grid), dim3(NTHREADS), args, experts_lds_bytes(E, EI),
			     (hipStream_t)stream);
	if (rc != hipSuccess)
		return (int)rc;
	return (int)hipGetLastError();
}
