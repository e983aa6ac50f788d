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
 * A workgroup of NW waves computes a tile of JT experts x TT tokens.  Each
 * logit is the 8 AVX2 lane accumulators of dot_f32_f32 (matmul.c:91-105):
 * accumulator l adds x[k]*w[k] for k = l, l+8, l+16, ... in increasing k
 * with FMA (the tiled T>1 path of matmul.c:213-238 keeps the same
 * per-element order); then the tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))
 * of vector_avx2.h:126-132 and logit = fl(bias + dot) (matmul.c:24-32).
 * Lane (token, expert, l) runs accumulator l alone (8 lanes per logit, the
 * shortest chain); the tree is three lane shuffles.  For few tokens (one a
 * workgroup: more workgroups); k_router_b below takes many.
 *
 * Router rows and tokens stream through an LDS ring of NST stages of
 * RT_KC = 256 columns (one 1 KB row piece per wave-wide LDS-DMA load,
 * global_load_lds_dwordx4, issued from inline assembly so the K loop alone
 * decides what to wait for); rows are padded to RT_RS bytes so the reads of
 * one wave hit distinct banks.  Every workgroup of an expert block reads
 * the same router rows at the same time, so first each one pulls a slice of
 * the block into its XCD's L2 (workgroups are dealt round-robin over the 8
 * XCDs: slice (blockIdx.x / 8) % nsl), and the ring's loads then hit there.
 */
#define RT_KC 256
#define RT_RS (RT_KC * 4 + 32)


template <int JT, int NW> struct rt_geo {
	static constexpr int LPL = 8;                     /* lanes per logit */
	static constexpr int TPW = WAVE / (LPL * JT);     /* tokens per wave */
	static constexpr int TT = NW * TPW;               /* tokens per workgroup */
	static constexpr int ROWS = JT + TT;              /* LDS rows per stage */
	static constexpr int PER = ROWS / NW;             /* row loads per wave and stage */
	static constexpr int SSZ = ROWS * RT_RS;
	static constexpr int NST1 = 150 * 1024 / SSZ, NST2 = 63 / PER + 2;
	static constexpr int NST = NST1 < NST2 ? NST1 : NST2; /* ring stages */
	static_assert(ROWS % NW == 0 && TPW >= 1 && NST >= 3, "router tile geometry");
};

template <int JT, int NW>
__global__ __launch_bounds__(NW * WAVE) void k_router(const float *__restrict__ x,
						      const float *__restrict__ wr,
						      const float *__restrict__ bias,
						      float *__restrict__ logits, int T, int E, int NE)
{
	typedef rt_geo<JT, NW> RG;
	constexpr int NST = RG::NST;
	__shared__ __attribute__((aligned(16))) uint8_t ring[NST * RG::SSZ + 1024];
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
	const int t0 = blockIdx.x * RG::TT, j0 = blockIdx.y * JT;
	const int tw = lane / (RG::LPL * JT), jl = (lane / RG::LPL) % JT, sub = lane % RG::LPL;
	const int tl = wave * RG::TPW + tw; /* token row of the tile */
	const int t = t0 + tl, j = j0 + jl;
	const int ns = E / RT_KC;
	const u32 l0 = (u32)(uintptr_t)(const __attribute__((address_space(3))) char *)ring;

	/* this workgroup's slice of the expert block, into L2: one 4-byte piece
	 * per 128-byte line, landing in a scratch kilobyte of LDS */
	{
		const int nrow = min(JT, NE - j0);
		const int nlines = nrow * E / 32;
		const int nsl = max(1, min(16, (int)gridDim.x / 8)), sl = (blockIdx.x / 8) % nsl;
		const float *blk = wr + (size_t)j0 * E;
		for (int q = wave; q * WAVE < nlines / nsl; q += NW) {
			const int line = sl + nsl * min(q * WAVE + lane, nlines / nsl - 1);
			dma_dwordx4(blk, (u32)line * 128u, l0 + (u32)(NST * RG::SSZ));
		}
	}

	/* row loads of this wave: rows wave, wave + NW, ... of [w rows | x rows];
	 * rows past NE or T repeat the last one (their results are not kept) */
	u32 roff[RG::PER];
	bool isw[RG::PER];
#pragma unroll
	for (int q = 0; q < RG::PER; q++) {
		const int r = wave + NW * q;
		isw[q] = r < JT;
		const int src = isw[q] ? min(j0 + r, NE - 1) : min(t0 + r - JT, T - 1);
		roff[q] = (u32)((size_t)src * E * 4 + 16 * lane);
	}
	auto issue = [&](int s) {
		const u32 st = l0 + (u32)((s % NST) * RG::SSZ);
#pragma unroll
		for (int q = 0; q < RG::PER; q++)
			dma_dwordx4((isw[q] ? wr : x) + (size_t)s * RT_KC, roff[q],
				 st + (u32)((wave + NW * q) * RT_RS));
	};

	float acc = 0.0f;
#pragma unroll
	for (int s = 0; s < NST - 1; s++)
		if (s < ns)
			issue(s);
	for (int s = 0; s < ns; s++) {
		if (s + NST - 2 < ns)
			wait_vm<(NST - 2) * RG::PER>();
		else
			wait_vm<0>();
		__syncthreads(); /* stage s landed for every wave; stage s-1 is free */
		if (s + NST - 1 < ns)
			issue(s + NST - 1);
		const uint8_t *st = ring + (s % NST) * RG::SSZ;
		const float *wrow = (const float *)(st + jl * RT_RS) + sub;
		const float *xrow = (const float *)(st + (JT + tl) * RT_RS) + sub;
		/* all 64 operand reads of the stage go out before the chain, one
		 * LDS latency per stage */
		float xs[RT_KC / 8], ws[RT_KC / 8];
#pragma unroll
		for (int i = 0; i < RT_KC / 8; i++) {
			xs[i] = xrow[8 * i];
			ws[i] = wrow[8 * i];
		}
#pragma unroll
		for (int i = 0; i < RT_KC / 8; i++)
			acc = __builtin_fmaf(xs[i], ws[i], acc);
	}
	/* lane l holds a_l: (a_l + a_l+4), then pairs, then the two halves */
	float v = acc;
	v = v + __shfl_xor(v, 4, 8);
	v = v + __shfl_xor(v, 2, 8);
	const float d = v + __shfl_xor(v, 1, 8);
	if (sub == 0 && t < T && j < NE)
		logits[(size_t)t * NE + j] = (bias ? bias[j] : 0.0f) + d;
}

/*
 * Many tokens: tiles of 16 experts x 8 tokens (RB_JT x RB_TT), 256 threads.
 * Lane (chain l = lane % 8, expert pair ep = lane / 8) of wave w runs
 * accumulator l of tokens 2w, 2w + 1 against experts 2ep, 2ep + 1: four
 * logits' chain l, so each LDS dword a lane reads feeds two FMAs (a lane
 * that ran four chains of one logit read two per FMA).  Chain l's values of
 * a row piece are every eighth dword (l, l + 8, ...): read in pairs
 * (ds_read2_b32).  Rows are padded to RB_RS bytes (260 dwords: row r starts
 * in bank 4r mod 32), so the 64 w addresses of a wave's read hit 32
 * distinct banks per half-wave and the x reads are broadcasts.  The chains
 * and the tree are the ones k_router forms: the same logits, bit for bit.
 * A 4-stage ring (3 in flight) starts computing sooner than a deeper one.
 * A stage takes ~0.8 us with or without its loads (timed by stamping a
 * copy whose stages all compute from one loaded stage): the LDS reads, at
 * one wave per SIMD, bound it.
 */
#define RB_JT 16
#define RB_TT 8
#define RB_RS (RT_KC * 4 + 16)
#define RB_NST 4

__global__ __launch_bounds__(256) void k_router_b(const float *__restrict__ x,
						  const float *__restrict__ wr,
						  const float *__restrict__ bias,
						  float *__restrict__ logits, int T, int E, int NE)
{
	constexpr int ROWS = RB_JT + RB_TT, NW = 4, PER = ROWS / NW, SSZ = ROWS * RB_RS;
	static_assert(ROWS % NW == 0 && RB_RS % 16 == 0 && (RB_RS / 4) % 32 == 4, "router tile");
	__shared__ __attribute__((aligned(16))) uint8_t ring[RB_NST * SSZ + 1024];
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
	const int l = lane & 7, ep = lane >> 3;
	const int t0 = blockIdx.x * RB_TT, j0 = blockIdx.y * RB_JT;
	const int ns = E / RT_KC;
	const u32 l0 = (u32)(uintptr_t)(const __attribute__((address_space(3))) char *)ring;

	/* this workgroup's slice of the expert block, into L2 (as k_router) */
	{
		const int nrow = min(RB_JT, NE - j0);
		const int nlines = nrow * E / 32;
		const int nsl = max(1, min(16, (int)gridDim.x / 8)), sl = (blockIdx.x / 8) % nsl;
		const float *blk = wr + (size_t)j0 * E;
		for (int q = wave; q * WAVE < nlines / nsl; q += NW) {
			const int line = sl + nsl * min(q * WAVE + lane, nlines / nsl - 1);
			dma_dwordx4(blk, (u32)line * 128u, l0 + (u32)(RB_NST * SSZ));
		}
	}

	/* row loads of this wave: rows wave, wave + NW, ... of [w rows | x rows];
	 * rows past NE or T repeat the last one (their results are not kept) */
	u32 roff[PER];
	bool isw[PER];
#pragma unroll
	for (int q = 0; q < PER; q++) {
		const int r = wave + NW * q;
		isw[q] = r < RB_JT;
		const int src = isw[q] ? min(j0 + r, NE - 1) : min(t0 + r - RB_JT, T - 1);
		roff[q] = (u32)((size_t)src * E * 4 + 16 * lane);
	}
	auto issue = [&](int s) {
		const u32 st = l0 + (u32)((s % RB_NST) * SSZ);
#pragma unroll
		for (int q = 0; q < PER; q++)
			dma_dwordx4((isw[q] ? wr : x) + (size_t)s * RT_KC, roff[q],
				    st + (u32)((wave + NW * q) * RB_RS));
	};

	float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}}; /* [token][expert] */
#pragma unroll
	for (int s = 0; s < RB_NST - 1; s++)
		if (s < ns)
			issue(s);
	for (int s = 0; s < ns; s++) {
		if (s + RB_NST - 2 < ns)
			wait_vm<(RB_NST - 2) * PER>();
		else
			wait_vm<0>();
		__syncthreads(); /* stage s landed for every wave; stage s-1 is free */
		if (s + RB_NST - 1 < ns)
			issue(s + RB_NST - 1);
		const uint8_t *st = ring + (s % RB_NST) * SSZ;
		const float *xr = (const float *)(st + (RB_JT + 2 * wave) * RB_RS) + l;
		const float *wv = (const float *)(st + 2 * ep * RB_RS) + l;
		/* the stage's 32 steps of the chain in batches of 4, double
		 * buffered: batch b + 1's reads go out before batch b's FMAs (a
		 * batch read then used at once left the LDS idle during the FMAs
		 * and the VALU idle during the reads) */
		float xa[2][4], wa[2][4], xb[2][4], wb[2][4];
		auto rd = [&](int b, float (&xs)[2][4], float (&ws)[2][4])
				  __attribute__((always_inline)) {
#pragma unroll
			for (int i = 0; i < 4; i++)
#pragma unroll
				for (int r = 0; r < 2; r++) {
					xs[r][i] = xr[r * (RB_RS / 4) + 8 * (4 * b + i)];
					ws[r][i] = wv[r * (RB_RS / 4) + 8 * (4 * b + i)];
				}
		};
		auto fm = [&](const float (&xs)[2][4], const float (&ws)[2][4])
				  __attribute__((always_inline)) {
#pragma unroll
			for (int i = 0; i < 4; i++)
#pragma unroll
				for (int tt = 0; tt < 2; tt++)
#pragma unroll
					for (int ee = 0; ee < 2; ee++)
						acc[tt][ee] = __builtin_fmaf(xs[tt][i], ws[ee][i], acc[tt][ee]);
		};
		rd(0, xa, wa);
#pragma unroll
		for (int b = 0; b < RT_KC / 32; b += 2) {
			rd(b + 1, xb, wb);
			fm(xa, wa);
			if (b + 2 < RT_KC / 32)
				rd(b + 2, xa, wa);
			fm(xb, wb);
		}
	}
	/* lane l holds a_l of each logit: (a_l + a_l+4), then pairs, then the halves */
#pragma unroll
	for (int tt = 0; tt < 2; tt++)
#pragma unroll
		for (int ee = 0; ee < 2; ee++) {
			float v = acc[tt][ee];
			v = v + __shfl_xor(v, 4, 8);
			v = v + __shfl_xor(v, 2, 8);
			const float d = v + __shfl_xor(v, 1, 8);
			const int t = t0 + 2 * wave + tt, j = j0 + 2 * ep + ee;
			if (l == 0 && t < T && j < NE)
				logits[(size_t)t * NE + j] = (bias ? bias[j] : 0.0f) + d;
		}
}

/* ------------------------------------------------------------------ */
/* softmax + top-k, one wave per token (wave_softmax_topk)             */
/* ------------------------------------------------------------------ */

/* rows [r0, r1) of x (E floats each) rounded to f16 into xh, NT threads */
template <int NT>
__device__ static inline void rows_to_f16(const float *x, _Float16 *xh, int r0, int r1, int E)
{
	typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
	const size_t n4 = (size_t)(r1 - r0) * E / 4, o4 = (size_t)r0 * E / 4;
	/* eight loads of a thread in flight at once (one per iteration waited
	 * a round trip each) */
	for (size_t i0 = threadIdx.x; i0 < n4; i0 += 8 * NT) {
		float4 v[8];
#pragma unroll
		for (int u = 0; u < 8; u++)
			if (i0 + u * NT < n4)
				v[u] = ((const float4 *)x)[o4 + i0 + u * NT];
#pragma unroll
		for (int u = 0; u < 8; u++)
			if (i0 + u * NT < n4) {
				half4_t h = {(_Float16)v[u].x, (_Float16)v[u].y, (_Float16)v[u].z,
					     (_Float16)v[u].w};
				((half4_t *)xh)[o4 + i0 + u * NT] = h;
			}
	}
}

__global__ __launch_bounds__(64) void k_softmax_topk(const float *__restrict__ logits,
						     float *__restrict__ probs,
						     u32 *__restrict__ ids,
						     float *__restrict__ wout,
						     int NE, int K, int renorm,
						     const float *__restrict__ x,
						     _Float16 *__restrict__ xh, int E)
{
	if (xh)
		rows_to_f16<64>(x, xh, blockIdx.x, blockIdx.x + 1, E);
	__shared__ float sp[MOE_MAX_NE];
	__shared__ u32 sid[MOE_MAX_TOPK];
	__shared__ float sw[MOE_MAX_TOPK];
	const int t = blockIdx.x;
	wave_softmax_topk(logits + (size_t)t * NE, probs ? probs + (size_t)t * NE : NULL,
			  ids + (size_t)t * K, wout + (size_t)t * K, NE, K, renorm, sp, sid, sw,
			  threadIdx.x);
}

/* NE <= 64: one wave per token, expert i in lane i, four tokens per
 * workgroup (softmax64 / rank_part64 / topk_finish64: the same arithmetic
 * and slots as wave_softmax_topk) */
__global__ __launch_bounds__(256) void k_softmax_topk64(const float *__restrict__ logits,
							float *__restrict__ probs,
							u32 *__restrict__ ids,
							float *__restrict__ wout, int T, int NE,
							int K, int renorm,
							const float *__restrict__ x,
							_Float16 *__restrict__ xh, int E)
{
	if (xh) { /* the f16 tokens, split over the whole grid */
		const int rows = (T + (int)gridDim.x - 1) / (int)gridDim.x;
		const int r0 = min((int)blockIdx.x * rows, T), r1 = min(r0 + rows, T);
		rows_to_f16<256>(x, xh, r0, r1, E);
	}
	if ((int)blockIdx.x * 4 >= T)
		return;
	__shared__ uint64_t s_tab[32];
	__shared__ __attribute__((aligned(16))) uint64_t s_key[4][WAVE];
	__shared__ u32 s_id[4][MOE_MAX_TOPK];
	__shared__ float s_w[4][MOE_MAX_TOPK];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int t = blockIdx.x * 4 + wave;
	const float logit = t < T && lane < NE ? logits[(size_t)t * NE + lane] : 0.0f;
	if (threadIdx.x < 32)
		s_tab[threadIdx.x] = moe_exp2_tab[threadIdx.x];
	__syncthreads();
	if (t >= T)
		return;
	uint64_t key;
	const float p = softmax64(logit, NE, s_tab, lane, key);
	if (probs && lane < NE)
		probs[(size_t)t * NE + lane] = p;
	s_key[wave][lane] = key;
	WAVE_SYNC();
	const int rank = rank_part64(s_key[wave], WAVE, key);
	topk_finish64(rank, p, ids + (size_t)t * K, wout + (size_t)t * K, NE, K, renorm,
		      s_id[wave], s_w[wave], lane);
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

/* four output columns per thread; the loads of up to 8 slots (and their
 * K-chunks) are issued together, then added in slot order */
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ ypart,
						 const float *__restrict__ w,
						 float *__restrict__ out, int K, int E,
						 int kchunks)
{
	const int t = blockIdx.y;
	const int i = 4 * (blockIdx.x * 256 + threadIdx.x);
	if (i >= E)
		return;
	float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
	/* slots s0 .. s0 + ns - 1 (ns <= NS), their K chunks added in chunk
	 * order, KB chunks' loads in flight at a time (one chunk per round trip
	 * held Mixtral's eight-chunk combine at ~8 us) */
	auto slots = [&](auto nsmax, auto kbc, int s0, int ns) {
		constexpr int NS = decltype(nsmax)::value, KB = decltype(kbc)::value;
		float4 y[NS];
#pragma unroll
		for (int s = 0; s < NS; s++)
			y[s] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
		for (int kc0 = 0; kc0 < kchunks; kc0 += KB) {
			float4 v[KB][NS];
#pragma unroll
			for (int j = 0; j < KB; j++)
#pragma unroll
				for (int s = 0; s < NS; s++)
					if (s < ns && kc0 + j < kchunks)
						v[j][s] = *(const float4 *)&ypart
							[(((size_t)t * K + s0 + s) * kchunks + kc0 + j) * E + i];
#pragma unroll
			for (int j = 0; j < KB; j++)
#pragma unroll
				for (int s = 0; s < NS; s++)
					if (s < ns && kc0 + j < kchunks) {
						if (kc0 + j == 0) {
							y[s] = v[j][s];
						} else {
							y[s].x += v[j][s].x;
							y[s].y += v[j][s].y;
							y[s].z += v[j][s].z;
							y[s].w += v[j][s].w;
						}
					}
		}
#pragma unroll
		for (int s = 0; s < NS; s++)
			if (s < ns) {
				const float inv = 1.0f / (w ? w[(size_t)t * K + s0 + s] : 1.0f);
				acc.x = acc.x + y[s].x / inv;
				acc.y = acc.y + y[s].y / inv;
				acc.z = acc.z + y[s].z / inv;
				acc.w = acc.w + y[s].w / inv;
			}
	};
	if (K <= 2) {
		slots(std::integral_constant<int, 2>(), std::integral_constant<int, 4>(), 0, K);
	} else {
		for (int s0 = 0; s0 < K; s0 += 8)
			slots(std::integral_constant<int, 8>(), std::integral_constant<int, 1>(), s0,
			      K - s0 < 8 ? K - s0 : 8);
	}
	float *o = &out[(size_t)t * E + i];
	if (((uintptr_t)out & 15) == 0) {
		*(float4 *)o = acc;
	} else { /* a caller's output that is not 16-byte aligned */
		o[0] = acc.x;
		o[1] = acc.y;
		o[2] = acc.z;
		o[3] = acc.w;
	}
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
				 float *logits, int T, int E, int NE, void *stream)
{
	if (T < 1 || NE < 1 || E % RT_KC || (size_t)NE * E * 4 > 0xffffffffull ||
	    (size_t)T * E * 4 > 0xffffffffull)
		return (int)hipErrorInvalidValue;
	/* tiles of 16 experts x 8 tokens, a lane one chain of 2 x 2 logits
	 * (k_router_b); for few tokens a chain a lane, tiles of 8 experts x 1
	 * token (more workgroups, but every token's workgroups load the router
	 * rows again).  Routing stage at NE = 64: one-token tiles 7.8 us up to
	 * T = 32, 11.5 at 64, 15.2 at 96, 39.6 at 320; 16x8 tiles with 4 chains
	 * of one logit a lane 12.4-13.4 us from T = 128 to 512; k_router_b at
	 * T = 512 10.6 us against 11.6 for those. */
	const int wide = ((T + 7) / 8) * ((NE + 15) / 16);
	if (NE > 8 && wide >= 36) {
		dim3 grid((T + RB_TT - 1) / RB_TT, (NE + RB_JT - 1) / RB_JT);
		hipLaunchKernelGGL(k_router_b, grid, dim3(256), 0, (hipStream_t)stream, x, wr, bias,
				   logits, T, E, NE);
	} else {
		dim3 grid(T, (NE + 7) / 8);
		hipLaunchKernelGGL((k_router<8, 1>), grid, dim3(64), 0, (hipStream_t)stream, x,
				   wr, bias, logits, T, E, NE);
	}
	return (int)hipGetLastError();
}

extern "C" int moe_launch_softmax_topk(const float *logits, float *probs, uint32_t *ids,
				       float *w, int T, int NE, int K, int renorm,
				       const float *x, void *xh, int E, void *stream)
{
	if (xh && E % 4)
		return (int)hipErrorInvalidValue;
	/* with f16 tokens: at least one workgroup per token (up to 256), so the
	 * copy is not held to the few CUs the routing needs */
	const int g64 = xh ? max((T + 3) / 4, min(T, 256)) : (T + 3) / 4;
	if (NE <= WAVE)
		hipLaunchKernelGGL(k_softmax_topk64, dim3(g64), dim3(256), 0,
				   (hipStream_t)stream, logits, probs, ids, w, T, NE, K, renorm, x,
				   (_Float16 *)xh, E);
	else
		hipLaunchKernelGGL(k_softmax_topk, dim3(T), dim3(64), 0, (hipStream_t)stream,
				   logits, probs, ids, w, NE, K, renorm, x, (_Float16 *)xh, E);
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
	if (E % 4)
		return (int)hipErrorInvalidValue;
	dim3 grid((E + 1023) / 1024, T);
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
