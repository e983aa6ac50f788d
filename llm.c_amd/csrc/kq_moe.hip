/*
 * kq_moe.hip - the MoE FFN's expert products on K-quant experts (Q4_K /
 * Q6_K, gate/up and down types chosen apart, as a Q4_K_M file mixes them),
 * bit for bit the reference's fused_ffn_silu (nn.c:449-539) in its default
 * -DQ8_DOT build:
 *
 *   k_kq_gateup  per (token, slot) pair p and rows j of expert ids[p]:
 *                g, u = dot_q8_quant(q8(x_t), gate/up row j) (the Q8_K
 *                integer dots of kquant.hip, the token quantized by each
 *                workgroup), h[p][j] = (g / (1 + expf(-g))) * u
 *                (nn.c:455-478; expf is glibc's, moe_expf.h)
 *   k_kq_down    y[p][i] = dot_f32_quant(h[p], down row i) (nn.c:483-492):
 *                the fp32 K-quant dot of quant.c:198-418 in its own order:
 *                accumulator l (of 8) takes elements l, l + 8, ... in
 *                increasing order with FMA, each weight fl(fl(d * sc) * q)
 *                - fl(dmin * m) (Q4_K) or fl((q - 32) * fl(d * sc)) (Q6_K),
 *                then the tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
 *
 * The combine (k_combine, y / (1/w) added in slot order) completes
 * olmoe.c:355-406 / llama.c:407-456, so the layer's outputs equal the
 * reference's bit for bit.
 *
 * Geometry.  k_kq_gateup: a workgroup per (pair, R = 128 / nb rows), a
 * thread per super-block of the R gate and R up rows (nb = E / 256 a row),
 * the block sums meet in LDS and a thread per row runs the sequential fp32
 * steps.  k_kq_down: 8 lanes per down row (lane l holds accumulator l), 32
 * rows per workgroup; the rows' super-blocks come through LDS in chunks of
 * KD_CB (contiguous runs, coalesced) with the matching KD_CB * 256 values
 * of h[p].
 *
 * Bound: HBM.  Algorithmic bytes per call: per pair, 2 * EI rows of E
 * columns and E rows of EI columns in their block types, plus x and h.
 */
#include "kq_device.h"

#define KG_THREADS 256
#define KD_THREADS 256
#define KD_ROWS 32 /* down rows a workgroup takes: 8 lanes each */
#define KD_CB 4    /* super-blocks of every row a chunk stages */
#define KC_DOTS 64 /* (row, pair) dots of a k_kq_down_combine workgroup: 8 lanes each */
#define KC_CB 4    /* d_ff super-blocks k_kq_down_combine stages (whole 8-byte steps: 4 * 210) */
#define KC_MAXP 8  /* pairs of a k_kq_down_combine call (a power of two: it divides KC_DOTS) */
#define KC_HPAD 8  /* floats between two pairs' staged h (banks apart) */

/* ------------------------------------------------------------------ */
/* gate/up                                                              */
/* ------------------------------------------------------------------ */

/*
 * Block b < 2 * R * nb of the workgroup: matrix b / (R * nb) (0 gate, 1 up),
 * row j0 + (b % (R * nb)) / nb, super-block b % nb.  Records (4 words: the
 * scale products and integer sums) per block in LDS, rows padded to nb + 1.
 */
template <int WT>
__global__ __launch_bounds__(KG_THREADS) void k_kq_gateup(
	const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up, size_t gu_stride,
	const u32 *__restrict__ ids, const float *__restrict__ x, float *__restrict__ h, int K,
	int E, int EI, int R)
{
	/* the token's Q8_K blocks, rows padded by one int: a wave's lanes read
	 * up to 16 blocks at the same offset, which then fall in distinct banks
	 * (a 64-int stride put them all in one) */
	constexpr int QS = 65, BS = 17;
	__shared__ int s_q8[32 * QS]; /* E <= 8192 */
	__shared__ float s_d[32];
	__shared__ int s_bs[32 * BS];
	__shared__ int s_rec[4][512]; /* 2 R (nb + 1) <= 512 for R * nb <= 128 */
	constexpr int BY = kqb<WT>::BYTES, DW = WT == 3 ? 36 : 53;
	const int p = blockIdx.y, t = p / K, nb = E / 256;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int j0 = blockIdx.x * R, RB = R * nb, rs = nb + 1;
	const size_t rb = (size_t)nb * BY;
	const size_t eo = (size_t)ids[p] * gu_stride;

	/* the weights first (one block per thread), then the token */
	u32 w[DW];
	const int b = tid < 2 * RB ? tid : 0;
	const int mat = b / RB, rl = (b % RB) / nb, sb = b % nb;
	const int row = min(j0 + rl, EI - 1);
	const uint8_t *blk = (mat ? up : gate) + eo + (size_t)row * rb + (size_t)sb * BY;
	if constexpr (WT == 3)
		load_dwords<36>(blk, w);
	else
		kg_load<53>(blk, w);
	/* the wave's token blocks (nb <= 32: at most 8 a wave), loaded together */
	float4 xv[8];
#pragma unroll
	for (int u = 0; u < 8; u++) {
		const int i = wave + u * (KG_THREADS / WAVE);
		if (i < nb)
			xv[u] = ((const float4 *)(x + (size_t)t * E + (size_t)i * 256))[lane];
	}
#pragma unroll
	for (int u = 0; u < 8; u++) {
		const int i = wave + u * (KG_THREADS / WAVE);
		if (i >= nb)
			break;
		const float4 v = xv[u];
		float d;
		int bs;
		const u32 q = kg_q8k(v, lane, &d, &bs);
		s_q8[i * QS + lane] = (int)q;
		if (lane % 4 == 0)
			s_bs[i * BS + lane / 4] = bs;
		if (lane == 0)
			s_d[i] = d;
	}
	__syncthreads();
	if (tid < 2 * RB) {
		float dsc, dmn = 0.0f;
		int sumi, msum = 0;
		if constexpr (WT == 3)
			kg_q4k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi, dmn, msum);
		else
			kg_q6k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi);
		const int slot = (mat * R + rl) * rs + sb;
		((float *)s_rec[0])[slot] = dsc;
		s_rec[1][slot] = sumi;
		((float *)s_rec[2])[slot] = dmn;
		s_rec[3][slot] = msum;
	}
	__syncthreads();
	/* thread r < R: row j0 + r, the reference's sequential steps for gate and
	 * up (dot_q4_K_q8_K returns acc + acc_m, dot_q6_K_q8_K acc) */
	if (tid < R && j0 + tid < EI) {
		float v[2];
#pragma unroll
		for (int m = 0; m < 2; m++) {
			const int o = (m * R + tid) * rs;
			float acc = 0.0f, acc_m = 0.0f;
			for (int i = 0; i < nb; i++) {
				acc = fmaf(((const float *)s_rec[0])[o + i], (float)s_rec[1][o + i], acc);
				if constexpr (WT == 3)
					acc_m = fmaf(((const float *)s_rec[2])[o + i], (float)s_rec[3][o + i],
						     acc_m);
			}
			v[m] = WT == 3 ? acc + acc_m : acc;
		}
		const float g = v[0];
		h[(size_t)p * EI + j0 + tid] = (g / (1.0f + moe_expf(-g))) * v[1];
	}
}

/* ------------------------------------------------------------------ */
/* down                                                                 */
/* ------------------------------------------------------------------ */

/*
 * Workgroup (row block r0 = blockIdx.x * KD_ROWS, pair p): wave w holds rows
 * r0 + 8w .. r0 + 8w + 7, lane 8k + l accumulator l of row r0 + 8w + k.
 * Each chunk of KD_CB super-blocks of all 32 rows goes to LDS (row r's run
 * is contiguous: KD_CB * BY bytes at row r, block c0), the 8 lanes of a row
 * then walk its blocks in order.
 */
template <int WT>
__global__ __launch_bounds__(KD_THREADS) void k_kq_down(const uint8_t *__restrict__ down,
						      size_t dn_stride, const u32 *__restrict__ ids,
						      const float *__restrict__ h, float *__restrict__ y,
						      int E, int EI)
{
	constexpr int BY = kqb<WT>::BYTES;
	constexpr int RUN = KD_CB * BY; /* bytes of one row's run (a multiple of 8) */
	__shared__ __attribute__((aligned(16))) float s_h[KD_CB * 256]; /* the chunk's h */
	__shared__ __attribute__((aligned(16))) uint8_t s_w[KD_ROWS * RUN];
	const int p = blockIdx.y, nb = EI / 256;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int l = lane & 7, rk = wave * 8 + lane / 8; /* row of the block */
	const int r0 = blockIdx.x * KD_ROWS;
	const size_t rb = (size_t)nb * BY;
	const uint8_t *base = down + (size_t)ids[p] * dn_stride;

	/* a chunk's 32 runs, 8 bytes a thread per step (runs are 2-byte aligned
	 * for Q6_K: dword pairs from the aligned address, realigned), and its h,
	 * into registers: every load goes out before any is stored (a loop that
	 * stored each before the next load waited ~13 round trips a chunk), and
	 * the next chunk's go out while this one's dots run */
	constexpr int NIT = (KD_ROWS * (RUN / 8) + KD_THREADS - 1) / KD_THREADS;
	constexpr int NH = (KD_CB * 64 + KD_THREADS - 1) / KD_THREADS;
	u32 v[NIT][3], shv[NIT];
	float4 hv[NH];
	auto load_chunk = [&](int c0) {
		const int run = min(KD_CB, nb - c0) * BY, cb = min(KD_CB, nb - c0);
#pragma unroll
		for (int it = 0; it < NIT; it++) {
			const int e = tid + it * KD_THREADS;
			const int r = e / (RUN / 8), o = 8 * (e % (RUN / 8));
			shv[it] = 0;
			if (e < KD_ROWS * (RUN / 8) && o < run) {
				const int row = min(r0 + r, E - 1);
				const uint8_t *src = base + (size_t)row * rb + (size_t)c0 * BY + o;
				const u32 sh = (u32)((uintptr_t)src & 3);
				const u32 *a = (const u32 *)(src - sh);
				v[it][0] = a[0];
				v[it][1] = a[1];
				v[it][2] = a[2];
				shv[it] = sh;
			}
		}
#pragma unroll
		for (int u = 0; u < NH; u++) {
			const int i = tid + u * KD_THREADS;
			if (i < cb * 64)
				hv[u] = ((const float4 *)(h + (size_t)p * EI + (size_t)c0 * 256))[i];
		}
	};
	float acc = 0.0f;
	load_chunk(0);
	for (int c0 = 0; c0 < nb; c0 += KD_CB) {
		const int cb = min(KD_CB, nb - c0);
		const int run = cb * BY;
		__syncthreads(); /* the previous chunk's readers are done */
#pragma unroll
		for (int u = 0; u < NH; u++) {
			const int i = tid + u * KD_THREADS;
			if (i < cb * 64)
				((float4 *)s_h)[i] = hv[u];
		}
#pragma unroll
		for (int it = 0; it < NIT; it++) {
			const int e = tid + it * KD_THREADS;
			const int r = e / (RUN / 8), o = 8 * (e % (RUN / 8));
			if (e < KD_ROWS * (RUN / 8) && o < run)
				*(uint2 *)(s_w + r * RUN + o) =
					make_uint2(__builtin_amdgcn_alignbyte(v[it][1], v[it][0], shv[it]),
						   __builtin_amdgcn_alignbyte(v[it][2], v[it][1], shv[it]));
		}
		__syncthreads();
		if (c0 + KD_CB < nb)
			load_chunk(c0 + KD_CB);
		for (int k = 0; k < cb; k++) {
			const uint8_t *blk = s_w + rk * RUN + k * BY;
			if constexpr (WT == 3)
				kd_q4k(blk, s_h + k * 256, l, acc);
			else
				kd_q6k(blk, s_h + k * 256, l, acc);
		}
	}
	/* vector_reduce_sum's tree: lanes l and l + 4, then l and l + 2, then 0
	 * and 1 (each add is one fp32 addition; which operand comes first does
	 * not change it) */
	acc = acc + __shfl_xor(acc, 4, 8);
	acc = acc + __shfl_xor(acc, 2, 8);
	acc = acc + __shfl_xor(acc, 1, 8);
	if (l == 0 && r0 + rk < E)
		y[(size_t)p * E + r0 + rk] = acc;
}

/*
 * k_kq_down with its chunks streamed through an LDS ring (KD_NS stages,
 * KD_NS - 1 chunks in flight) by LDS-DMA loads that the kernel counts
 * itself, where every row's run starts 4-byte aligned (nb * BY % 4 == 0:
 * Q4_K always, Q6_K for an even number of super-blocks a row).  k_kq_down
 * holds one chunk in flight in registers (the compiler waits for all of a
 * thread's loads before it stores any, so more chunks in registers do not
 * overlap); at Mixtral's shape a workgroup (one per CU) then waited out
 * most of a round trip per chunk.  A stage: the 32 rows' runs as 16-byte
 * pieces (KD_NPR a row, row stride KD_NPR * 16 in LDS; the last piece
 * reads up to 8 bytes past the run, inside the row's successor or the
 * weights' slack) and the chunk's h.  The same dots in the same order.
 */
#define KD_NS 4

template <int WT>
__global__ __launch_bounds__(KD_THREADS) void k_kq_down_r(const uint8_t *__restrict__ down,
							size_t dn_stride, const u32 *__restrict__ ids,
							const float *__restrict__ h, float *__restrict__ y,
							int E, int EI)
{
	constexpr int BY = kqb<WT>::BYTES;
	constexpr int RUN = KD_CB * BY;                         /* bytes of a row's run */
	constexpr int NPR = (RUN + 15) / 16;                    /* 16-byte pieces a row */
	constexpr int RSL = NPR * 16;                           /* LDS row stride */
	constexpr int NPC = KD_ROWS * NPR;                      /* pieces a chunk */
	constexpr int JB = (NPC + KD_THREADS - 1) / KD_THREADS; /* weight loads a thread */
	constexpr int SW = JB * KD_THREADS * 16;                /* weight bytes a stage */
	constexpr int SSZ = SW + KD_CB * 256 * 4;               /* + the chunk's h */
	constexpr int LOADS = JB + 1;                           /* loads a wave a stage */
	static_assert(KD_CB * 64 == KD_THREADS, "one h piece a thread");
	static_assert((KD_NS - 2) * LOADS < 64, "vmcnt");
	__shared__ __attribute__((aligned(16))) uint8_t ring[KD_NS * SSZ];
	const int p = blockIdx.y, nb = EI / 256, nch = (nb + KD_CB - 1) / KD_CB;
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int l = lane & 7, rk = wave * 8 + lane / 8; /* row of the block */
	const int r0 = blockIdx.x * KD_ROWS;
	const u32 rb = (u32)(nb * BY);
	const uint8_t *base = down + (size_t)ids[p] * dn_stride;
	const float *hp = h + (size_t)p * EI;
	const u32 l0 = __builtin_amdgcn_readfirstlane(lds_addr(ring));
	/* piece f = (wave * JB + j) * 64 + lane of a chunk: row f / NPR, piece
	 * f % NPR; pieces past NPC read row r0's first piece (never used) */
	u32 woff[JB], wpc[JB];
#pragma unroll
	for (int j = 0; j < JB; j++) {
		const int f = (wave * JB + j) * WAVE + lane;
		const int row = min(r0 + (f < NPC ? f / NPR : 0), E - 1);
		woff[j] = (u32)row * rb;
		wpc[j] = f < NPC ? 16u * (u32)(f % NPR) : 0u;
	}
	auto issue = [&](int s) {
		const u32 st = l0 + (u32)((s % KD_NS) * SSZ);
		/* a partial last chunk's pieces past its blocks re-read the run's
		 * first piece (read past the run, they would leave the last row) */
		const u32 lim = (u32)(min(KD_CB, nb - s * KD_CB) * BY);
#pragma unroll
		for (int j = 0; j < JB; j++)
			dma_dwordx4(base, woff[j] + (u32)s * RUN + (wpc[j] < lim ? wpc[j] : 0u),
				    st + (u32)((wave * JB + j) * WAVE * 16));
		/* h piece tid of the chunk, clamped into the row's EI values
		 * (a partial last chunk's pieces past the row are never used) */
		const int cb = min(KD_CB, nb - s * KD_CB);
		const int g = min(tid, cb * 64 - 1);
		dma_dwordx4(hp, (u32)(s * KD_CB * 256 + 4 * g) * 4u, st + SW + (u32)(wave * WAVE * 16));
	};
#pragma unroll
	for (int s = 0; s < KD_NS - 1; s++)
		if (s < nch)
			issue(s);
	float acc = 0.0f;
	for (int s = 0; s < nch; s++) {
		if (s + KD_NS - 2 < nch)
			wait_vm<(KD_NS - 2) * LOADS>();
		else
			wait_vm<0>();
		__syncthreads(); /* chunk s landed for every wave; slot s - 1 is free */
		if (s + KD_NS - 1 < nch)
			issue(s + KD_NS - 1);
		const uint8_t *st = ring + (s % KD_NS) * SSZ;
		const float *sh = (const float *)(st + SW);
		const int cb = min(KD_CB, nb - s * KD_CB);
		for (int k = 0; k < cb; k++) {
			const uint8_t *blk = st + rk * RSL + k * BY;
			if constexpr (WT == 3)
				kd_q4k(blk, sh + k * 256, l, acc);
			else
				kd_q6k(blk, sh + k * 256, l, acc);
		}
	}
	/* vector_reduce_sum's tree, as k_kq_down */
	acc = acc + __shfl_xor(acc, 4, 8);
	acc = acc + __shfl_xor(acc, 2, 8);
	acc = acc + __shfl_xor(acc, 1, 8);
	if (l == 0 && r0 + rk < E)
		y[(size_t)p * E + r0 + rk] = acc;
}

/* ------------------------------------------------------------------ */
/* down and combine of a decode-sized call                              */
/* ------------------------------------------------------------------ */

/*
 * The second launch of the decode-sized K-quant layer where d_ff is at most
 * KC_CB super-blocks (the first, k_kq_route_gateup in moe_decode.hip,
 * routes and writes h[P][EI], ids and weights): workgroup b takes output
 * rows r0 = b * RB .. r0 + RB - 1 (RB = KC_DOTS / P) for every pair p = t *
 * K + k, one (row, pair) dot per 8 lanes, the same dot and order as
 * k_kq_down (dot_f32_quant of h[p] with down row r of expert ids[p]); then
 * out[t][r] = sum over the slots k in order of y / (1/w), as k_combine adds
 * them (olmoe.c:401-403, tensor.c:334-353, 435-456).  The rows' super-blocks
 * and every pair's h are staged in LDS once.  Dots go pair-major (dot d:
 * pair d / RB, row d % RB), so a wave's eight dots read at most two pairs'
 * h, whose LDS rows are padded apart by KC_HPAD floats (other banks).  The h
 * loads (independent of the routing) go out before the wait for the ids.
 * Longer d_ff takes k_kq_down and k_combine after the first launch: there
 * every workgroup would re-read all pairs' h chunk by chunk.
 *
 * Dynamic LDS: P rows of KC_CB * 256 + KC_HPAD floats of h, then KC_DOTS
 * runs of KC_CB super-blocks.
 */
template <int WT, int PM>
__global__ __launch_bounds__(KC_DOTS * 8) void k_kq_down_combine(
	const uint8_t *__restrict__ down, size_t dn_stride, const u32 *__restrict__ ids,
	const float *__restrict__ wts, const float *__restrict__ h, float *__restrict__ out, int T,
	int K, int E, int EI)
{
	constexpr int NTH = KC_DOTS * 8; /* 8 lanes per dot */
	constexpr int BY = kqb<WT>::BYTES;
	constexpr int RUN = KC_CB * BY; /* bytes of one dot's run */
	static_assert(RUN % 8 == 0, "a run is staged in 8-byte steps");
	constexpr int HS = KC_CB * 256 + KC_HPAD; /* floats of one pair's staged h */
	extern __shared__ __attribute__((aligned(16))) float kc_lds[];
	__shared__ float s_y[KC_DOTS];
	/* each pair's expert as a byte offset: a pointer read from LDS would be
	 * a generic one, and its flat loads wait on the LDS counter */
	__shared__ size_t s_eo[KC_MAXP];
	__shared__ float s_wt[KC_MAXP];
	const int P = T * K, RB = KC_DOTS / P, nb = EI / 256;
	float *s_h = kc_lds;                              /* [P][HS] */
	uint8_t *s_w = (uint8_t *)(kc_lds + (size_t)P * HS); /* [KC_DOTS][RUN] */
	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int l = lane & 7, dk = wave * 8 + lane / 8; /* this lane's dot */
	const int r0 = blockIdx.x * RB;
	const size_t rb = (size_t)nb * BY, run = (size_t)nb * BY;

	constexpr int NIT = (KC_DOTS * (RUN / 8) + NTH - 1) / NTH;
	/* PM >= P: the pairs' h a thread loads */
	constexpr int NH = (PM * KC_CB * 64 + NTH - 1) / NTH;
	/* a native vector type: an array of the float4 struct stays in scratch
	 * memory */
	typedef float f4v __attribute__((ext_vector_type(4)));
	f4v hv[NH];
#pragma unroll
	for (int u = 0; u < NH; u++) {
		/* float4 i of the pairs' P x KC_CB * 64, clamped into the d_ff
		 * (the stores below skip the clamped ones) */
		const int i = tid + u * NTH;
		const int p = min(i / (KC_CB * 64), P - 1), q = min(i % (KC_CB * 64), nb * 64 - 1);
		hv[u] = ((const f4v *)(h + (size_t)p * EI))[q];
	}
	if (tid < P) { /* each pair's expert and slot weight, once */
		s_eo[tid] = (size_t)ids[tid] * dn_stride;
		s_wt[tid] = wts[tid];
	}
	__syncthreads();
	/* every weight load goes out before any is stored (as k_kq_down) */
	u32 v[NIT][3], shv[NIT];
#pragma unroll
	for (int it = 0; it < NIT; it++) {
		const int e = tid + it * NTH;
		const int d = e / (RUN / 8), o = 8 * (e % (RUN / 8));
		shv[it] = 0;
		if (e < KC_DOTS * (RUN / 8) && o < (int)run) {
			const int row = r0 + d % RB, p = d / RB;
			const uint8_t *src = down + s_eo[p] + (size_t)row * rb + o;
			const u32 sh = (u32)((uintptr_t)src & 3);
			const u32 *a = (const u32 *)(src - sh);
			v[it][0] = a[0];
			v[it][1] = a[1];
			v[it][2] = a[2];
			shv[it] = sh;
		}
	}
#pragma unroll
	for (int u = 0; u < NH; u++) {
		const int i = tid + u * NTH;
		const int p = i / (KC_CB * 64), q = i % (KC_CB * 64);
		if (p < P && q < nb * 64)
			((f4v *)(s_h + (size_t)p * HS))[q] = hv[u];
	}
#pragma unroll
	for (int it = 0; it < NIT; it++) {
		const int e = tid + it * NTH;
		const int d = e / (RUN / 8), o = 8 * (e % (RUN / 8));
		if (e < KC_DOTS * (RUN / 8) && o < (int)run)
			*(uint2 *)(s_w + d * RUN + o) =
				make_uint2(__builtin_amdgcn_alignbyte(v[it][1], v[it][0], shv[it]),
					   __builtin_amdgcn_alignbyte(v[it][2], v[it][1], shv[it]));
	}
	__syncthreads();
	const float *hp = s_h + (size_t)(dk / RB) * HS;
	float acc = 0.0f;
	for (int k = 0; k < nb; k++) {
		const uint8_t *blk = s_w + dk * RUN + k * BY;
		if constexpr (WT == 3)
			kd_q4k(blk, hp + k * 256, l, acc);
		else
			kd_q6k(blk, hp + k * 256, l, acc);
	}
	/* vector_reduce_sum's tree, as k_kq_down */
	acc = acc + __shfl_xor(acc, 4, 8);
	acc = acc + __shfl_xor(acc, 2, 8);
	acc = acc + __shfl_xor(acc, 1, 8);
	if (l == 0) /* (row, pair) in the combine's order */
		s_y[(dk % RB) * P + dk / RB] = acc;
	__syncthreads();
	if (tid < RB * T) {
		const int r = tid / T, t = tid % T;
		float o = 0.0f;
		for (int k = 0; k < K; k++) {
			const int p = t * K + k;
			const float inv = 1.0f / s_wt[p];
			o = o + s_y[r * P + p] / inv;
		}
		out[(size_t)t * E + r0 + r] = o;
	}
}

/* ------------------------------------------------------------------ */
/* host side                                                            */
/* ------------------------------------------------------------------ */

extern "C" int moe_kq_layer_supported(int gt, int dt, size_t E, size_t EI)
{
	const int gk = gt == 3 || gt == 5, dk = dt == 3 || dt == 5;
	return gk && dk && E % 256 == 0 && EI % 256 == 0 && E <= 8192 && E / 256 <= 128 &&
	       EI <= 16384;
}

extern "C" int moe_launch_kq_gateup(int gt, const uint8_t *gate, const uint8_t *up,
				    size_t gu_stride, const u32 *ids, const float *x, float *h,
				    int P, int K, int E, int EI, void *stream)
{
	const int nb = E / 256, R = max(1, 128 / nb);
	const dim3 grid((EI + R - 1) / R, P);
	hipStream_t s = (hipStream_t)stream;
	if (gt == 3)
		hipLaunchKernelGGL(k_kq_gateup<3>, grid, dim3(KG_THREADS), 0, s, gate, up, gu_stride,
				   ids, x, h, K, E, EI, R);
	else
		hipLaunchKernelGGL(k_kq_gateup<5>, grid, dim3(KG_THREADS), 0, s, gate, up, gu_stride,
				   ids, x, h, K, E, EI, R);
	return (int)hipGetLastError();
}

extern "C" int moe_launch_kq_down(int dt, const uint8_t *down, size_t dn_stride, const u32 *ids,
				  const float *h, float *y, int P, int E, int EI, void *stream)
{
	const dim3 grid((E + KD_ROWS - 1) / KD_ROWS, P);
	hipStream_t s = (hipStream_t)stream;
	const int nb = EI / 256;
	/* the LDS ring where every row's run is 4-byte aligned and the
	 * offsets of one expert's rows fit 32 bits */
	const int bytes = dt == 3 ? 144 : 210;
	const bool ring = (nb * bytes) % 4 == 0 && dn_stride % 4 == 0 && ((uintptr_t)down & 3) == 0 &&
			  dn_stride + 4096 < 0xffffffffull;
	if (dt == 3 && ring)
		hipLaunchKernelGGL(k_kq_down_r<3>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids,
				   h, y, E, EI);
	else if (ring)
		hipLaunchKernelGGL(k_kq_down_r<5>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids,
				   h, y, E, EI);
	else if (dt == 3)
		hipLaunchKernelGGL(k_kq_down<3>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids, h,
				   y, E, EI);
	else
		hipLaunchKernelGGL(k_kq_down<5>, grid, dim3(KD_THREADS), 0, s, down, dn_stride, ids, h,
				   y, E, EI);
	return (int)hipGetLastError();
}

/* the down + combine launch of a decode-sized call of P = T * K pairs: P a
 * power of two up to KC_MAXP (it divides KC_DOTS), every output row of E in
 * one workgroup's block of KC_DOTS / P rows, d_ff at most KC_CB super-blocks */
extern "C" int moe_kq_down_combine_ok(size_t T, size_t K, size_t E, size_t EI)
{
	const size_t P = T * K;
	return P >= 1 && P <= KC_MAXP && (P & (P - 1)) == 0 && E % (KC_DOTS / P) == 0 &&
	       EI % 256 == 0 && EI >= 256 && EI <= 256 * KC_CB;
}

extern "C" int moe_launch_kq_down_combine(int dt, const uint8_t *down, size_t dn_stride,
					  const u32 *ids, const float *w, const float *h,
					  float *out, int T, int K, int E, int EI, void *stream)
{
	if (!moe_kq_down_combine_ok((size_t)T, (size_t)K, (size_t)E, (size_t)EI) ||
	    (dt != 3 && dt != 5))
		return (int)hipErrorInvalidValue;
	const int P = T * K, RB = KC_DOTS / P;
	const size_t lds = (size_t)P * (KC_CB * 256 + KC_HPAD) * sizeof(float) +
			   (size_t)KC_DOTS * KC_CB * (dt == 3 ? 144 : 210);
	const dim3 grid(E / RB);
	hipStream_t s = (hipStream_t)stream;
	const int pm = P <= 1 ? 1 : P <= 2 ? 2 : P <= 4 ? 4 : 8;
	const void *fn = NULL;
#define KCPICK(D_, PM_)                                                       \
	if (dt == D_ && pm == PM_)                                            \
		fn = (const void *)k_kq_down_combine<D_, PM_>;
	KCPICK(3, 1) KCPICK(3, 2) KCPICK(3, 4) KCPICK(3, 8)
	KCPICK(5, 1) KCPICK(5, 2) KCPICK(5, 4) KCPICK(5, 8)
#undef KCPICK
	static_assert(KC_MAXP == 8, "instances cover pair bounds 1, 2, 4, 8");
	void *args[] = {&down, &dn_stride, &ids, &w, &h, &out, &T, &K, &E, &EI};
	hipError_t rc = hipLaunchKernel(fn, grid, dim3(KC_DOTS * 8), args, lds, s);
	if (rc != hipSuccess)
		return (int)rc;
	return (int)hipGetLastError();
}
