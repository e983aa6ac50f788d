/*
 * Decode-sized MoE FFN layer (T*K <= 64) in one launch: k_moe_decode.
 *
 * Every workgroup (G of them, four per CU) runs:
 *
 *  1. routing.  Workgroup j < NE computes router logit j for every token
 *     with the 8-lane FMA chains of dot_f32_f32 (matmul.c:91-105), fed from
 *     LDS-transposed copies of router row j and the token, and writes it into
 *     NREP replicas of the logit table, each entry tagged with this launch's
 *     epoch.  Every workgroup then polls its own replica (lane j of a wave
 *     polls expert j of a token; the loads that see the epoch deliver the
 *     logits) and runs softmax + top-k (+ renorm) itself (nn.c:221-308,
 *     llama.c:422-427): no second hop, no hot line.
 *  2. expert items, statically assigned: item i runs on workgroup i % G, in
 *     increasing i.  Items are gate/up tiles (8 rows of gate and up of the
 *     expert in slot p: h[p][row] = silu(gate.x) * (up.x), nn.c:460-478), each
 *     ending with its tile flag, then down tiles (16 rows of down over one
 *     K-chunk of h[p], nn.c:490-492).  A down tile issues its weight loads,
 *     then waits for the flags of the gate/up tiles covering its K-chunk.
 *     The workgroup holding the last down tile of a (token, row block) waits
 *     for the others and combines the slots in order: out += y / (1/w)
 *     (olmoe.c:401-403).
 *  3. epoch.  Each workgroup raises a start flag once it has read the epoch
 *     word; workgroup 0, when done with its items, checks them and advances
 *     the epoch for the next launch (which starts after this one drains).
 *
 * Synchronisation uses no read-modify-write: same-address device atomics
 * serialise (~0.1 us each), so producers write epoch-tagged flags (one word
 * per producing wave) and consumers poll them.  Dependencies point only to
 * items with smaller indices, which every workgroup processes first, so with
 * all G workgroups resident (G is the occupancy limit) every wait ends.
 * Waits are bounded regardless; one that runs out sets an error word instead
 * of hanging.
 *
 * Data produced by another workgroup in the same launch (logits, h, partial
 * y) is written with device-coherent stores (agent-scope relaxed atomics:
 * `sc1` on gfx950, written through the per-XCD L2) and read with
 * device-coherent loads; a producer waits for its stores to complete
 * (s_waitcnt) before raising its flag.  Agent-scope release/acquire fences
 * are avoided: on gfx950 they write back / invalidate a whole XCD L2.
 *
 * Weights stay in GGUF block layout.  A lane owns one segment of a row:
 * Q8_0 one 34-byte block (9 dwords loaded from the 4-byte aligned window
 * that holds it, 32 columns), Q4_0 a pair of 18-byte blocks (9 dwords, 64
 * columns), and keeps the matching activations in registers.
 */
#include "moe_device.h"

#define NTHREADS 256
#define GU_ROWS 8
#define DN_ROWS 16
#define NREP 64 /* == WAVE: one replica per lane of the writing wave */
#define COMBINE_MAX 1024 /* floats of LDS for the combiner's partials */

struct DecodeArgs {
	const float *x;
	const float *router;
	const float *bias;
	const uint8_t *gate, *up, *down;
	size_t gu_stride, dn_stride;
	u32 *ids_out;
	float *w_out;
	float *h;
	float *ypart;
	float *out;
	u32 *sync;
	int T, E, EI, NE, K, renorm, kch;
	int n_gu, n_dn;
	int off_start, off_rep, off_hf;
	int rep_stride; /* u64 entries between replicas (a multiple of 512: 4 KB) */
};

#define SPIN_LIMIT (1 << 20)

/* device-coherent accesses (global_{load,store} ... sc1) */
__device__ static inline void st_dev(float *p, float v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline void st_dev_u32(u32 *p, u32 v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline void st_dev_u64(uint64_t *p, uint64_t v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline float ld_dev(const float *p)
{
	return __hip_atomic_load((float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline u32 ld_dev_u32(const u32 *p)
{
	return __hip_atomic_load((u32 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline uint64_t ld_dev_u64(const uint64_t *p)
{
	return __hip_atomic_load((uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ static inline void backoff(int &step)
{
	switch (step) {
	case 0: __builtin_amdgcn_s_sleep(1); break;
	case 1: __builtin_amdgcn_s_sleep(2); break;
	case 2: __builtin_amdgcn_s_sleep(4); break;
	default: __builtin_amdgcn_s_sleep(8); break;
	}
	step += step < 3;
}

/*
 * The whole workgroup waits until n flags starting at f all equal `epoch`.
 * Each thread checks n / NTHREADS of them per round.
 */
__device__ static inline void wait_flags(const u32 *f, int n, u32 epoch, u32 *err)
{
	__shared__ int s_ok;
	int step = 0;
	for (int round = 0;; round++) {
		bool ok = true;
		for (int i = threadIdx.x; i < n; i += NTHREADS)
			ok &= ld_dev_u32(&f[i]) == epoch;
		if (threadIdx.x == 0)
			s_ok = 1;
		__syncthreads();
		if (!ok)
			s_ok = 0;
		__syncthreads();
		if (s_ok)
			return;
		if (round >= SPIN_LIMIT) {
			if (threadIdx.x == 0)
				st_dev_u32(err, 1u);
			return;
		}
		backoff(step);
		__syncthreads();
	}
}

/* ---------------------------------------------------------------------- */
/* segments                                                               */
/* ---------------------------------------------------------------------- */

template <int WT> struct segq;

/* Q8_0: one block per lane.  Block s of a row starts at byte 34s; the 36-byte
 * window starting at (34s & ~3) holds it: scale in bytes 0-1 of the window
 * (even s) or 2-3 (odd s), quants right after. */
template <> struct segq<1> {
	static constexpr int DW = 9, COLS = 32;
	__device__ static inline const uint8_t *win(const uint8_t *row, int s)
	{
		return row + ((34 * s) & ~3);
	}
	/* block sums of x: one block per lane */
	__device__ static inline void xsum(const float (&x)[32], float (&xs)[2])
	{
		xs[0] = sum32(x);
		xs[1] = 0.0f;
	}
	__device__ static inline float dot(const u32 (&d)[9], const float (&x)[32], int s,
					   const float (&xs)[2])
	{
		u32 q[8];
		const bool odd = s & 1; /* quants at byte 4 (odd) or 2 (even) of the window */
#pragma unroll
		for (int k = 0; k < 8; k++)
			q[k] = odd ? d[k + 1] : __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		return block_dot_q8_0(q, odd ? d[0] >> 16 : d[0], x, xs[0]);
	}
};

/* Q4_0: a pair of blocks per lane, 36 bytes at 36s (quant.c:126-155). */
template <> struct segq<2> {
	static constexpr int DW = 9, COLS = 64;
	__device__ static inline const uint8_t *win(const uint8_t *row, int s)
	{
		return row + 36 * s;
	}
	__device__ static inline void xsum(const float (&x)[64], float (&xs)[2])
	{
		xs[0] = sum32(x);
		xs[1] = sum32(x + 32);
	}
	__device__ static inline float dot(const u32 (&d)[9], const float (&x)[64], int,
					   const float (&xs)[2])
	{
		return seg_dot_q4_0(d, x, xs[0], xs[1]);
	}
};

template <int COLS>
__device__ static inline void lds_seg(const float *s, int seg, float (&x)[COLS])
{
	const float4 *s4 = (const float4 *)(s + seg * (COLS + 4));
#pragma unroll
	for (int i = 0; i < COLS / 4; i++) {
		float4 v = s4[i];
		x[4 * i + 0] = v.x;
		x[4 * i + 1] = v.y;
		x[4 * i + 2] = v.z;
		x[4 * i + 3] = v.w;
	}
}

/* n floats from global into LDS, COLS-float segments padded by 4 floats */
template <int COLS>
__device__ static inline void stage_seg(float *s, const float *g, int n)
{
	const float4 *g4 = (const float4 *)g;
	for (int i = threadIdx.x; i < n / 4; i += NTHREADS) {
		int k = 4 * i;
		*(float4 *)(s + (k / COLS) * (COLS + 4) + k % COLS) = g4[i];
	}
}

/* ---------------------------------------------------------------------- */
/* routing                                                                */
/* ---------------------------------------------------------------------- */

/* copy n floats, element k -> dst[(k & 7) * RS + (k >> 3)] */
__device__ static inline void stage_transposed(float *dst, const float *src, int n, int RS)
{
	const float4 *s4 = (const float4 *)src;
	for (int i = threadIdx.x; i < n / 4; i += NTHREADS) {
		float4 v = s4[i];
		int k = 4 * i;
		dst[((k + 0) & 7) * RS + ((k + 0) >> 3)] = v.x;
		dst[((k + 1) & 7) * RS + ((k + 1) >> 3)] = v.y;
		dst[((k + 2) & 7) * RS + ((k + 2) >> 3)] = v.z;
		dst[((k + 3) & 7) * RS + ((k + 3) >> 3)] = v.w;
	}
}

/* acc = fma(x[k], w[k], acc) over k = 0, 8, 16, ... of one transposed row
 * pair (E8 floats each).  The chain is 256 dependent FMAs for E = 2048, so
 * its LDS operands are fetched two batches (of 16 FMAs) ahead. */
struct chain_batch {
	float4 x[4], w[4];
	__device__ inline void load(const float4 *xr, const float4 *wr, int b)
	{
#pragma unroll
		for (int u = 0; u < 4; u++) {
			x[u] = xr[4 * b + u];
			w[u] = wr[4 * b + u];
		}
	}
	__device__ inline float run(float acc) const
	{
#pragma unroll
		for (int u = 0; u < 4; u++) {
			acc = __builtin_fmaf(x[u].x, w[u].x, acc);
			acc = __builtin_fmaf(x[u].y, w[u].y, acc);
			acc = __builtin_fmaf(x[u].z, w[u].z, acc);
			acc = __builtin_fmaf(x[u].w, w[u].w, acc);
		}
		return acc;
	}
};

__device__ static inline float router_chain(const float *xrow, const float *wrow, int E8)
{
	const float4 *xr = (const float4 *)xrow, *wr = (const float4 *)wrow;
	const int nb = E8 / 16; /* batches of 16 FMAs */
	chain_batch A, B, C;
	float acc = 0.0f;
	A.load(xr, wr, 0);
	if (nb > 1)
		B.load(xr, wr, 1);
	for (int b = 0; b < nb; b += 3) {
		if (b + 2 < nb)
			C.load(xr, wr, b + 2);
		acc = A.run(acc);
		if (b + 1 >= nb)
			break;
		if (b + 3 < nb)
			A.load(xr, wr, b + 3);
		acc = B.run(acc);
		if (b + 2 >= nb)
			break;
		if (b + 4 < nb)
			B.load(xr, wr, b + 4);
		acc = C.run(acc);
	}
	return acc;
}

/* router row j for every token, published into every replica by wave 0;
 * prev_epoch (the launch's epoch minus one, valid in thread 0) is consumed
 * only after the chain, so its load is in flight meanwhile */
__device__ static void router_row(const DecodeArgs &a, int j, u32 prev_epoch, float *lds)
{
	const int E = a.E, E8 = E / 8, RS = E8 + 4;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	float *sw = lds;          /* [8][RS] router row, transposed */
	float *sx = lds + 8 * RS; /* [8][RS] token, transposed */
	__shared__ float s_logit;
	uint64_t *rep = (uint64_t *)(a.sync + a.off_rep);

	stage_transposed(sw, a.router + (size_t)j * E, E, RS);
	for (int t = 0; t < a.T; t++) {
		stage_transposed(sx, a.x + (size_t)t * E, E, RS);
		__syncthreads();
		if (wave == 0) {
			/* lane l < 8 replays AVX2 lane l: elements l, l+8, ... in order */
			const int l = lane & 7;
			float acc = router_chain(sx + l * RS, sw + l * RS, E8);
			acc = acc + __shfl_xor(acc, 4, 8);
			acc = acc + __shfl_xor(acc, 2, 8);
			acc = acc + __shfl_xor(acc, 1, 8);
			if (lane == 0)
				s_logit = (a.bias ? a.bias[j] : 0.0f) + acc;
		}
		__syncthreads();
		if (wave == 0) { /* NREP == WAVE: lane r writes replica r */
			const u32 ep = __shfl(prev_epoch, 0, WAVE) + 1;
			const uint64_t v = ((uint64_t)ep << 32) | __builtin_bit_cast(u32, s_logit);
			st_dev_u64(&rep[(size_t)lane * a.rep_stride + (size_t)t * a.NE + j], v);
		}
		__syncthreads();
	}
}

/*
 * Routing of every token from this workgroup's replica: wave w takes tokens
 * w, w+4, ...; lane j polls entry (t, j) until the whole row carries the
 * epoch (one hop: the loads that see the epoch also deliver the logits), then
 * the wave runs softmax + top-k (+ renorm) into s_ids/s_w [T*K].
 */
__device__ static void route_local(const DecodeArgs &a, u32 epoch, float *lds, u32 *s_ids,
				   float *s_w, const uint64_t *s_tab)
{
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const uint64_t *rep = (const uint64_t *)(a.sync + a.off_rep) +
			      (size_t)(blockIdx.x % NREP) * a.rep_stride;
	float *scr = lds + wave * (MOE_MAX_NE + 2 * MOE_MAX_TOPK);
	for (int t = wave; t < a.T; t += NTHREADS / WAVE) { /* NE <= 64: one expert per lane */
		const uint64_t *row = rep + (size_t)t * a.NE;
		float logit = 0.0f;
		int step = 0;
		for (int round = 0;; round++) {
			const uint64_t v = lane < a.NE ? ld_dev_u64(&row[lane]) : (uint64_t)epoch << 32;
			if (__all((u32)(v >> 32) == epoch)) {
				logit = __builtin_bit_cast(float, (u32)v);
				break;
			}
			if (round >= SPIN_LIMIT) {
				if (lane == 0)
					st_dev_u32(a.sync + MOE_SYNC_ERR_WORD, 1u);
				break;
			}
			backoff(step);
		}
		wave_softmax_topk64(logit, s_ids + t * a.K, s_w + t * a.K, a.NE, a.K, a.renorm, s_tab,
				    scr, (u32 *)(scr + MOE_MAX_NE), scr + MOE_MAX_NE + MOE_MAX_TOPK,
				    lane);
	}
	__syncthreads();
}

/* ---------------------------------------------------------------------- */
/* expert items                                                           */
/* ---------------------------------------------------------------------- */

template <int WT, int CD> struct down_geo {
	static constexpr int RPS = WAVE / CD, RW = DN_ROWS / 4, NS = RW / RPS;
	static constexpr int CHUNK = CD * segq<WT>::COLS; /* columns of one K-chunk */
	static constexpr int CD_SEGS = CD;                /* segments of one K-chunk */
};

/* issue the weight loads of down item d (they do not depend on h) */
template <int WT, int CD>
__device__ static inline void down_load(const DecodeArgs &a, int d, const u32 *s_ids,
					u32 (&dd)[down_geo<WT, CD>::NS][9])
{
	typedef segq<WT> S;
	typedef down_geo<WT, CD> DG;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int nrb = a.E / DN_ROWS;
	const int p = d / (a.kch * nrb), rem = d % (a.kch * nrb);
	const int kc = rem / nrb, rbk = rem % nrb;
	const int row0 = rbk * DN_ROWS + wave * DG::RW;
	const int seg = lane % CD, sub = lane / CD;
	const size_t rb = (size_t)(a.EI / MOE_QK) * (WT == 1 ? 34 : 18);
	const uint8_t *D = S::win(a.down + (size_t)s_ids[p] * a.dn_stride, kc * CD + seg);
#pragma unroll
	for (int s2 = 0; s2 < DG::NS; s2++)
		load_dwords<S::DW>(D + (size_t)(row0 + s2 * DG::RPS + sub) * rb, dd[s2]);
}

/* the weights of one gate/up tile in registers */
template <int WT, int CG> struct gu_regs {
	static constexpr int RPS = WAVE / CG, RW = GU_ROWS / 4, NS = RW / RPS;
	u32 g[NS][segq<WT>::DW], u[NS][segq<WT>::DW];
};

/* issue the weight loads of gate/up tile g */
template <int WT, int CG>
__device__ static inline void gateup_load(const DecodeArgs &a, int g, const u32 *s_ids,
					  gu_regs<WT, CG> &r)
{
	typedef segq<WT> S;
	typedef gu_regs<WT, CG> R;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int tiles = a.EI / GU_ROWS;
	const int p = g / tiles, tile = g % tiles;
	const int row0 = tile * GU_ROWS + wave * R::RW;
	const int e = (int)s_ids[p];
	const int seg = lane % CG, sub = lane / CG;
	const size_t rb = (size_t)(a.E / MOE_QK) * (WT == 1 ? 34 : 18);
	const uint8_t *G = S::win(a.gate + (size_t)e * a.gu_stride, seg);
	const uint8_t *U = S::win(a.up + (size_t)e * a.gu_stride, seg);
#pragma unroll
	for (int s2 = 0; s2 < R::NS; s2++) {
		const size_t ro = (size_t)(row0 + s2 * R::RPS + sub) * rb;
		load_dwords<S::DW>(G + ro, r.g[s2]);
		load_dwords<S::DW>(U + ro, r.u[s2]);
	}
}

/* Gate/up tile g with its weights in r: h[p][rows] = silu(gate.x) * (up.x)
 * (the stores; the flag follows in gateup_flag) */
template <int WT, int CG>
__device__ static void gateup_compute(const DecodeArgs &a, int g, float *sx, int &staged,
				      const gu_regs<WT, CG> &r, const uint64_t *s_tab)
{
	typedef segq<WT> S;
	typedef gu_regs<WT, CG> R;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int tiles = a.EI / GU_ROWS;
	const int p = g / tiles, tile = g % tiles;
	const int row0 = tile * GU_ROWS + wave * R::RW;
	const int t = p / a.K;
	const int seg = lane % CG, sub = lane / CG;
	if (staged != t) {
		__syncthreads(); /* earlier readers of sx are done */
		stage_seg<S::COLS>(sx, a.x + (size_t)t * a.E, a.E);
		__syncthreads();
		staged = t;
	}
	float xr[S::COLS], xs[2];
	lds_seg<S::COLS>(sx, seg, xr);
	S::xsum(xr, xs);
#pragma unroll
	for (int s2 = 0; s2 < R::NS; s2++) {
		const int row = row0 + s2 * R::RPS + sub;
		const float gv = group_sum<CG>(S::dot(r.g[s2], xr, seg, xs));
		const float uv = group_sum<CG>(S::dot(r.u[s2], xr, seg, xs));
		if (seg == 0)
			st_dev(&a.h[(size_t)p * a.EI + row],
			       (gv / (1.0f + moe_expf_tab(-gv, s_tab))) * uv);
	}
	/* keep the h stores ahead of any load the caller issues next */
	asm volatile("" ::: "memory");
}

/*
 * The flag of gate/up tile g, raised once its h stores have completed: wait
 * until at most N vector memory operations are outstanding.  They retire in
 * issue order, so N = the loads issued after the stores (the next item's
 * weights, in flight while this wait covers only older operations).
 */
template <int N>
__device__ static inline void gateup_flag(const DecodeArgs &a, int g, u32 epoch)
{
	static_assert(N >= 0 && N < 64, "vmcnt is six bits");
	__builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
	__syncthreads();
	if (threadIdx.x == 0)
		st_dev_u32(a.sync + a.off_hf + (size_t)g, epoch); /* p * tiles + tile == g */
}

/* n floats another workgroup produced in this launch, from global into LDS
 * (COLS-float segments padded by 4) */
template <int COLS>
__device__ static inline void stage_seg_dev(float *s, const float *g, int n)
{
	for (int i = threadIdx.x; i < n / 2; i += NTHREADS) {
		uint64_t v = ld_dev_u64((const uint64_t *)(g + 2 * i));
		int k = 2 * i;
		*(uint64_t *)(s + (k / COLS) * (COLS + 4) + k % COLS) = v;
	}
}

/* down item d with its weights already in dd: wait for the gate/up tiles of
 * its K-chunk of h[p], write partial y; the last contribution (in item order) of a (token, row
 * block) waits for the others and combines the slots in order */
template <int WT, int CD>
__device__ static void down_item(const DecodeArgs &a, int d, const float *s_w, float *sh,
				 float *sc, int &hchunk, u32 epoch,
				 const u32 (&dd)[down_geo<WT, CD>::NS][9])
{
	typedef segq<WT> S;
	typedef down_geo<WT, CD> DG;
	constexpr int TPC = DG::CHUNK / GU_ROWS; /* gate/up tiles per K-chunk */
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int nrb = a.E / DN_ROWS;
	const int p = d / (a.kch * nrb), rem = d % (a.kch * nrb);
	const int kc = rem / nrb, rbk = rem % nrb;
	const int t = p / a.K, slot = p % a.K;
	const int row0 = rbk * DN_ROWS + wave * DG::RW;
	const int seg = lane % CD, sub = lane / CD;
	const int ncontrib = a.K * a.kch, own = slot * a.kch + kc;
	const bool combiner = slot == a.K - 1 && kc == a.kch - 1;
	__shared__ float s_y[DN_ROWS];

	if (hchunk != p * a.kch + kc) { /* consecutive items mostly share the chunk */
		wait_flags(a.sync + a.off_hf + (size_t)p * (a.EI / GU_ROWS) + (size_t)kc * TPC, TPC,
			   epoch, a.sync + MOE_SYNC_ERR_WORD);
		stage_seg_dev<S::COLS>(sh, a.h + (size_t)p * a.EI + (size_t)kc * DG::CHUNK,
				       DG::CHUNK);
		__syncthreads();
		hchunk = p * a.kch + kc;
	}
	float xr[S::COLS], xs[2];
	lds_seg<S::COLS>(sh, seg, xr);
	S::xsum(xr, xs);
	/* partial y of (token, row block), contribution (slot, kc), tagged with
	 * the epoch so the combiner can poll the data itself */
	uint64_t *yq = (uint64_t *)a.ypart + ((size_t)t * nrb + rbk) * ncontrib * DN_ROWS;
#pragma unroll
	for (int s2 = 0; s2 < DG::NS; s2++) {
		const int r = wave * DG::RW + s2 * DG::RPS + sub;
		const float y = group_sum<CD>(S::dot(dd[s2], xr, kc * CD + seg, xs));
		if (seg == 0) {
			if (combiner)
				s_y[r] = y;
			else
				st_dev_u64(&yq[(size_t)own * DN_ROWS + r],
					   ((uint64_t)epoch << 32) | __builtin_bit_cast(u32, y));
		}
	}
	if (!combiner)
		return;
	/* the combiner: collect the other contributions, then add the slots in
	 * order, y = sum of its K-chunks in order, out += y / (1/w) */
	const int n = ncontrib * DN_ROWS; /* sc: [ncontrib][DN_ROWS] */
	__shared__ int s_ok;
	int step = 0;
	for (int round = 0;; round++) {
		bool ok = true;
		for (int i = threadIdx.x; i < n; i += NTHREADS) {
			if (i / DN_ROWS == own)
				continue;
			const uint64_t v = ld_dev_u64(&yq[i]);
			ok &= (u32)(v >> 32) == epoch;
			sc[i] = __builtin_bit_cast(float, (u32)v);
		}
		if (threadIdx.x == 0)
			s_ok = 1;
		__syncthreads();
		if (!ok)
			s_ok = 0;
		__syncthreads();
		if (s_ok)
			break;
		if (round >= SPIN_LIMIT) {
			if (threadIdx.x == 0)
				st_dev_u32(a.sync + MOE_SYNC_ERR_WORD, 1u);
			break;
		}
		backoff(step);
		__syncthreads();
	}
	if (threadIdx.x < DN_ROWS) {
		const int r = threadIdx.x;
		sc[own * DN_ROWS + r] = s_y[r];
		float acc = 0.0f;
		for (int s = 0; s < a.K; s++) {
			const size_t ps = (size_t)t * a.K + s;
			float y = sc[(s * a.kch) * DN_ROWS + r];
			for (int c = 1; c < a.kch; c++)
				y += sc[(s * a.kch + c) * DN_ROWS + r];
			acc = acc + y / (1.0f / s_w[ps]);
		}
		a.out[(size_t)t * a.E + rbk * DN_ROWS + r] = acc;
	}
}

/*
 * PIPE = 0: four workgroups per CU (<= 128 VGPRs), items run one after the
 * other (decode of one OLMoE token: one gate/up and one down item each).
 * PIPE = 1: two workgroups per CU (<= 256 VGPRs) and the weight loads of the
 * next item are in flight while the current one computes (Mixtral-sized
 * layers: several items per workgroup).
 */
template <int WT, int CG, int CD, int PIPE>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(PIPE ? 2 : 4,
									   PIPE ? 2 : 4)))
void k_moe_decode(DecodeArgs a)
{
	extern __shared__ float lds[];
	__shared__ u32 s_ids[MOE_FUSED_MAX_P];
	__shared__ float s_w[MOE_FUSED_MAX_P];
	__shared__ u32 s_epoch;
	__shared__ uint64_t s_tab[32];
	typedef segq<WT> S;

	if (threadIdx.x < 32)
		s_tab[threadIdx.x] = moe_exp2_tab[threadIdx.x];
	u32 prev_epoch = 0;
	if (threadIdx.x == 0)
		prev_epoch = ld_dev_u32(a.sync); /* consumed late: the load overlaps routing */
	if ((int)blockIdx.x < a.NE) {
		router_row(a, blockIdx.x, prev_epoch, lds);
		__syncthreads();
	}
	if (threadIdx.x == 0)
		s_epoch = prev_epoch + 1;
	__syncthreads();
	const u32 epoch = s_epoch;
	/* this workgroup has read the epoch word: workgroup 0 may advance it
	 * once every workgroup has said so */
	u32 *startf = a.sync + a.off_start;
	if (threadIdx.x == 0 && blockIdx.x != 0)
		st_dev_u32(&startf[blockIdx.x], epoch);
	route_local(a, epoch, lds, s_ids, s_w, s_tab);
	if (blockIdx.x == 0)
		for (int i = threadIdx.x; i < a.T * a.K; i += NTHREADS) {
			a.ids_out[i] = s_ids[i];
			a.w_out[i] = s_w[i];
		}

	float *sx = lds;                                       /* x, padded segments */
	float *sh = lds + (a.E / S::COLS) * (S::COLS + 4);     /* h chunk, padded */
	typedef down_geo<WT, CD> DG;
	float *sc = sh + DG::CD_SEGS * (S::COLS + 4);          /* combiner partials */
	int staged = -1, hchunk = -1;
	const int G = (int)gridDim.x;
	/* gate/up tiles cyclically (tile i on workgroup i % G); down tiles in
	 * contiguous blocks, so consecutive ones share their K-chunk of h.  Each
	 * workgroup runs its items in increasing index and every wait is for a
	 * smaller index, so with the grid resident every wait ends. */
	const int m = (a.n_dn + G - 1) / G;
	const int d0 = (int)blockIdx.x * m < a.n_dn ? (int)blockIdx.x * m : a.n_dn;
	const int d1 = d0 + m < a.n_dn ? d0 + m : a.n_dn;
	if (PIPE) {
		constexpr int NLD = 6 * gu_regs<WT, CG>::NS; /* loads of one gateup_load */
		gu_regs<WT, CG> A, B;
		int item = blockIdx.x;
		if (item < a.n_gu)
			gateup_load<WT, CG>(a, item, s_ids, A);
		if (item + G < a.n_gu)
			gateup_load<WT, CG>(a, item + G, s_ids, B);
		for (; item < a.n_gu; item += 2 * G) {
			gateup_compute<WT, CG>(a, item, sx, staged, A, s_tab);
			if (item + 2 * G < a.n_gu) {
				gateup_load<WT, CG>(a, item + 2 * G, s_ids, A);
				gateup_flag<NLD>(a, item, epoch);
			} else {
				gateup_flag<0>(a, item, epoch);
			}
			const int n1 = item + G;
			if (n1 >= a.n_gu)
				break;
			gateup_compute<WT, CG>(a, n1, sx, staged, B, s_tab);
			if (n1 + 2 * G < a.n_gu) {
				gateup_load<WT, CG>(a, n1 + 2 * G, s_ids, B);
				gateup_flag<NLD>(a, n1, epoch);
			} else {
				gateup_flag<0>(a, n1, epoch);
			}
		}
		u32 dA[DG::NS][9], dB[DG::NS][9];
		int d = d0;
		if (d < d1)
			down_load<WT, CD>(a, d, s_ids, dA);
		while (d < d1) {
			if (d + 1 < d1)
				down_load<WT, CD>(a, d + 1, s_ids, dB);
			down_item<WT, CD>(a, d, s_w, sh, sc, hchunk, epoch, dA);
			__syncthreads();
			if (++d >= d1)
				break;
			if (d + 1 < d1)
				down_load<WT, CD>(a, d + 1, s_ids, dA);
			down_item<WT, CD>(a, d, s_w, sh, sc, hchunk, epoch, dB);
			__syncthreads();
			++d;
		}
	} else {
		u32 dd[DG::NS][9];
		bool have_dd = false;
		for (int item = blockIdx.x; item < a.n_gu; item += G) {
			gu_regs<WT, CG> r;
			gateup_load<WT, CG>(a, item, s_ids, r);
			gateup_compute<WT, CG>(a, item, sx, staged, r, s_tab);
			gateup_flag<0>(a, item, epoch);
			/* the first down item's weights: issued only now, so they do not
			 * compete with the gate/up streams everyone is waiting for */
			if (item + G >= a.n_gu && d0 < d1) {
				down_load<WT, CD>(a, d0, s_ids, dd);
				have_dd = true;
			}
		}
		for (int d = d0; d < d1; d++) {
			if (!have_dd)
				down_load<WT, CD>(a, d, s_ids, dd);
			have_dd = false;
			down_item<WT, CD>(a, d, s_w, sh, sc, hchunk, epoch, dd);
			__syncthreads();
		}
	}

	/* workgroup 0 advances the epoch for the next launch once every
	 * workgroup has read it (they did so long ago: no wait in practice);
	 * the next launch starts only after this one has drained */
	if (blockIdx.x != 0)
		return;
	wait_flags(startf + 1, (int)gridDim.x - 1, epoch, a.sync + MOE_SYNC_ERR_WORD);
	if (threadIdx.x == 0)
		st_dev_u32(a.sync, epoch);
}

/* ---------------------------------------------------------------------- */

/* Q4_0 layers (Mixtral-sized) run the pipelined two-per-CU form */
template <int WT, int CG, int CD>
static const void *decode_fn()
{
	return (const void *)k_moe_decode<WT, CG, CD, WT == 2 ? 1 : 0>;
}

/* Q8_0: CG = E/32, CD from EI/32; Q4_0: CG = E/64, CD from EI/64 */
static const void *pick_decode(int wtype, int CG, int CD)
{
#define F3(W_, G, D)                                  \
	if (wtype == W_ && CG == G && CD == D)        \
		return decode_fn<W_, G, D>();
#define FD(W_, G) F3(W_, G, 16) F3(W_, G, 32) F3(W_, G, 64)
	FD(1, 32) FD(1, 64) FD(2, 32) FD(2, 64)
#undef FD
#undef F3
	return NULL;
}

static int seg_cols(int wtype)
{
	return wtype == 1 ? 32 : 64;
}

/* lanes per row: the largest power of two <= 64 dividing K / cols */
static int lanes_for(size_t K, int cols)
{
	size_t nseg = K / (size_t)cols;
	int c = 64;
	while (c > 1 && nseg % (size_t)c)
		c >>= 1;
	return c;
}

struct Geo {
	int CG, CD, kch;
	const void *fn;
};

static Geo geometry(int wtype, size_t E, size_t EI)
{
	Geo g;
	int cols = seg_cols(wtype);
	g.CG = lanes_for(E, cols);
	g.CD = lanes_for(EI, cols);
	g.kch = (int)(EI / (size_t)cols / (size_t)g.CD);
	g.fn = NULL;
	if (E % (size_t)cols || EI % (size_t)cols || E / (size_t)cols != (size_t)g.CG)
		return g; /* a gate/up row must fit one wave */
	g.fn = pick_decode(wtype, g.CG, g.CD);
	return g;
}

static size_t decode_lds_bytes(int wtype, size_t E, size_t EI, size_t T, size_t NE)
{
	int cols = seg_cols(wtype);
	Geo g = geometry(wtype, E, EI);
	size_t rt = (size_t)2 * 8 * (E / 8 + 4) * sizeof(float);
	size_t tk = (((T * NE + 15) & ~(size_t)15) + 4 * (MOE_MAX_NE + 2 * MOE_MAX_TOPK)) *
		    sizeof(float);
	/* x, one K-chunk of h, and the combiner's partials (K * kch * DN_ROWS
	 * <= COMBINE_MAX floats) */
	size_t ex = ((E / cols + g.CD) * (cols + 4) + COMBINE_MAX) * sizeof(float);
	size_t m = rt > tk ? rt : tk;
	return m > ex ? m : ex;
}

struct SyncLayout {
	size_t off_start, off_rep, off_hf, words, rep_stride;
};

static SyncLayout sync_layout(int wtype, size_t T, size_t K, size_t E, size_t EI, size_t NE,
			      int grid)
{
	Geo g = geometry(wtype, E, EI);
	SyncLayout s;
	s.rep_stride = (T * NE + 511) & ~(size_t)511;
	s.off_start = 1024;
	s.off_rep = s.off_start + (((size_t)grid + 1023) & ~(size_t)1023);
	s.off_hf = s.off_rep + (size_t)NREP * s.rep_stride * 2;
	s.words = s.off_hf + T * K * (EI / GU_ROWS);
	return s;
}

extern "C" int moe_fused_supported(int wtype, size_t E, size_t EI, size_t NE, size_t T,
				   size_t K)
{
	if (NE > WAVE || T * K > MOE_FUSED_MAX_P || E % DN_ROWS || EI % GU_ROWS || E % 256 ||
	    EI % 256)
		return 0;
	Geo g = geometry(wtype, E, EI);
	/* the combiner gathers K * kch contributions of DN_ROWS rows in LDS */
	if (K * (size_t)g.kch * DN_ROWS > COMBINE_MAX)
		return 0;
	return g.fn != NULL;
}

extern "C" int moe_fused_kchunks(int wtype, size_t EI)
{
	return geometry(wtype, 4096, EI).kch;
}

extern "C" size_t moe_fused_sync_words(int wtype, size_t T, size_t K, size_t E, size_t EI,
				       size_t NE, int grid)
{
	return sync_layout(wtype, T, K, E, EI, NE, grid).words;
}

extern "C" int moe_fused_grid(int wtype, size_t E, size_t EI, size_t NE)
{
	Geo g = geometry(wtype, E, EI);
	if (!g.fn)
		return 0;
	int dev = 0, ncu = 0, per = 0;
	if (hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		return 0;
	size_t lds = decode_lds_bytes(wtype, E, EI, MOE_FUSED_MAX_P, NE);
	if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, g.fn, NTHREADS, lds) != hipSuccess ||
	    per < 1)
		return 0;
	if (per > MOE_FUSED_WG_PER_CU)
		per = MOE_FUSED_WG_PER_CU;
	int grid = ncu * per;
	return grid >= (int)NE ? grid : 0; /* router rows need one workgroup each */
}

extern "C" int moe_launch_fused(int wtype, const float *x, const float *router,
				const float *bias, const uint8_t *gate, const uint8_t *up,
				const uint8_t *down, size_t gu_stride, size_t dn_stride,
				uint32_t *ids, float *w, float *h, float *ypart, float *out,
				uint32_t *sync, int T, int E, int EI, int NE, int K, int renorm,
				int grid, void *stream)
{
	Geo g = geometry(wtype, (size_t)E, (size_t)EI);
	if (!g.fn || grid < NE)
		return (int)hipErrorInvalidValue;
	SyncLayout sl = sync_layout(wtype, (size_t)T, (size_t)K, (size_t)E, (size_t)EI,
				    (size_t)NE, grid);
	DecodeArgs a;
	a.x = x;
	a.router = router;
	a.bias = bias;
	a.gate = gate;
	a.up = up;
	a.down = down;
	a.gu_stride = gu_stride;
	a.dn_stride = dn_stride;
	a.ids_out = ids;
	a.w_out = w;
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
	a.kch = g.kch;
	a.n_gu = T * K * (EI / GU_ROWS);
	a.n_dn = T * K * g.kch * (E / DN_ROWS);
	a.off_start = (int)sl.off_start;
	a.off_rep = (int)sl.off_rep;
	a.off_hf = (int)sl.off_hf;
	a.rep_stride = (int)sl.rep_stride;
	void *args[] = {&a};
	hipError_t rc = hipLaunchKernel(g.fn, dim3(grid), dim3(NTHREADS), args,
					decode_lds_bytes(wtype, (size_t)E, (size_t)EI, (size_t)T,
							 (size_t)NE),
					(hipStream_t)stream);
	if (rc != hipSuccess)
		return (int)rc;
	return (int)hipGetLastError();
}
