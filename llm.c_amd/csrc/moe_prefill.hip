/*
 * Prefill-sized MoE FFN layer: tokens sorted by expert, then grouped GEMMs
 * on the f16 matrix cores.
 *
 *   k_moe_sort     stable counting sort of the T*K (token, slot) pairs by
 *                  expert into m-tiles of PF_MT rows (the tail of each
 *                  expert's last tile is padding, row id -1), and the tile
 *                  table tile -> expert.
 *   k_pf_gateup    per (m-tile, 128 h columns): G = X Wg^T and U = X Wu^T
 *                  over d_model, h = silu(G) * U  (nn.c:460-478), stored f16
 *                  in sorted row order.
 *   k_pf_down      per (m-tile, 256 output columns): Y = H Wd^T over d_ff,
 *                  written fp32 to ypart[pair][E]; k_combine then adds the
 *                  slots of each token in order, out += y / (1/w)
 *                  (olmoe.c:401-403).
 *
 * The reference computes every (token, expert) product as its own fp32
 * dequant-dot (fused_ffn_silu per token, olmoe.c:364-395, quant.c:103-155).
 * Here the same products run as v_mfma_f32_32x32x16_f16 with fp32
 * accumulation: activations are rounded to f16, and each weight block is
 * dequantized to f16(d * q) in registers, one GGML block (32 k) feeding two
 * MFMAs.  The per-block scale stays inside the operand, so no per-block
 * rescaling of accumulators is needed (an int8 MFMA over 32-element blocks
 * would need ~32 VALU operations of rescaling per 32-cycle MFMA).  The
 * rounding of x and of d*q to f16 costs ~5e-4 relative L2 on the layer
 * output, within the 1e-3 the layer is held to.
 *
 * Operand layouts of v_mfma_f32_32x32x16_f16 (lane l, h = l / 32):
 *   A (32 x 16, rows m):   lane l holds A[l % 32][8h .. 8h+7]
 *   B (16 x 32, cols n):   lane l holds B[8h .. 8h+7][l % 32]
 *   D (32 x 32):           element j of lane l is D[8(j/4) + 4h + j%4][l % 32]
 * A 32-column block b of a weight row is split as: k-half 0 = elements
 * 8h..8h+7, k-half 1 = elements 16+8h..16+8h+7, so a lane needs quants
 * 8h..8h+7 and 16+8h..16+8h+7 (Q8_0) or packed bytes 8h..8h+7 (Q4_0: low
 * nibbles are elements 8h+i, high nibbles 16+8h+i) plus the block scale.
 */
#include "moe_device.h"

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

#define PF_MT 64            /* rows (pairs) per m-tile */
#define PF_KB 64            /* k per pipeline step: two blocks */
#define PF_THREADS 256
#define PF_LDA (PF_KB + 8)  /* halves per LDS row of the activation tile */
#define PF_GU_COLS 128      /* h columns per gate/up workgroup, 32 per wave */
#define PF_DN_COLS 256      /* output columns per down workgroup, 64 per wave */
#define SORT_THREADS 1024

/* ---------------------------------------------------------------------- */
/* sort                                                                    */
/* ---------------------------------------------------------------------- */

/*
 * One workgroup.  Pairs keep their order inside an expert (stable), so the
 * layout is a deterministic function of ids.  rows[] gets Tmax*PF_MT entries
 * (padding -1) and tile_e[] Tmax entries (-1 past the last tile): every
 * entry is rewritten on every call.
 *
 * Thread (e, c) = (tid % NE, tid / NE) owns expert e in chunk c of each
 * segment of SORT_SEG pairs (ids staged in LDS as bytes): it counts its
 * expert's pairs in the chunk, takes the exclusive sum of the counts of the
 * earlier chunks, and writes its pairs' rows in order.
 */
#define SORT_SEG 16384

__global__ __launch_bounds__(SORT_THREADS) void k_moe_sort(const u32 *__restrict__ ids, int P,
							   int NE, int Tmax,
							   int *__restrict__ rows,
							   int *__restrict__ tile_e)
{
	__shared__ int cnt[MOE_MAX_NE], toff[MOE_MAX_NE + 1], run[MOE_MAX_NE];
	__shared__ int ccnt[SORT_THREADS];
	__shared__ __attribute__((aligned(16))) uint8_t sid[SORT_SEG];
	const int tid = threadIdx.x;
	const int C = SORT_THREADS / NE; /* chunks per segment */
	const int e = tid % NE, c = tid / NE;
	const bool owner = c < C;

	for (int i = tid; i < NE; i += SORT_THREADS) {
		cnt[i] = 0;
		run[i] = 0;
	}
	__syncthreads();
	for (int p = tid; p < P; p += SORT_THREADS) {
		const u32 v = ids[p];
		if (v < (u32)NE) /* always, for ids from the top-k kernel */
			atomicAdd(&cnt[v], 1);
	}
	__syncthreads();
	if (tid < WAVE) { /* exclusive scan of tiles per expert, 4 experts per lane */
		const int lane = tid;
		int t4[4], s = 0;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int ex = 4 * lane + i;
			t4[i] = ex < NE ? (cnt[ex] + PF_MT - 1) / PF_MT : 0;
			s += t4[i];
		}
		int incl = s;
#pragma unroll
		for (int d = 1; d < WAVE; d <<= 1) {
			const int v = __shfl_up(incl, d, WAVE);
			if (lane >= d)
				incl += v;
		}
		int base = incl - s;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int ex = 4 * lane + i;
			if (ex < NE)
				toff[ex] = base;
			base += t4[i];
		}
		if (lane == WAVE - 1)
			toff[NE] = incl;
	}
	__syncthreads();
	const int ntiles = toff[NE];
	/* tile table and padding rows */
	for (int i = tid; i < Tmax * PF_MT; i += SORT_THREADS) {
		const int tile = i / PF_MT;
		int ex = -1;
		if (tile < ntiles) { /* largest ex with toff[ex] <= tile */
			int lo = 0, hi = NE - 1;
			while (lo < hi) {
				const int mid = (lo + hi + 1) >> 1;
				if (toff[mid] <= tile)
					lo = mid;
				else
					hi = mid - 1;
			}
			ex = lo;
		}
		if (i % PF_MT == 0)
			tile_e[tile] = ex;
		if (ex < 0 || i - toff[ex] * PF_MT >= cnt[ex])
			rows[i] = -1;
	}
	/* stable scatter, segment by segment */
	for (int s0 = 0; s0 < P; s0 += SORT_SEG) {
		const int S = P - s0 < SORT_SEG ? P - s0 : SORT_SEG;
		__syncthreads(); /* earlier readers of sid / ccnt are done */
		for (int i = tid; i < S; i += SORT_THREADS) {
			const u32 v = ids[s0 + i];
			sid[i] = v < (u32)NE ? (uint8_t)v : (uint8_t)255; /* NE <= 256 */
		}
		__syncthreads();
		const int L = (S + C - 1) / C;
		const int b0 = c * L, b1 = b0 + L < S ? b0 + L : S;
		int n = 0;
		if (owner)
			for (int i = b0; i < b1; i++)
				n += sid[i] == (uint8_t)e;
		ccnt[tid] = n;
		__syncthreads();
		if (owner) {
			int pos = toff[e] * PF_MT + run[e];
			for (int cc = 0; cc < c; cc++)
				pos += ccnt[cc * NE + e];
			for (int i = b0; i < b1; i++)
				if (sid[i] == (uint8_t)e)
					rows[pos++] = s0 + i;
		}
		__syncthreads();
		if (tid < NE) {
			int tot = 0;
			for (int cc = 0; cc < C; cc++)
				tot += ccnt[cc * NE + tid];
			run[tid] += tot;
		}
	}
}

/* ---------------------------------------------------------------------- */
/* weight operands                                                         */
/* ---------------------------------------------------------------------- */

/* two f16 (1024 + byte) from bytes sel of u, as selected by a v_perm pattern */
__device__ static inline half2_t magic2(u32 u, u32 sel)
{
	return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, sel));
}

/* 8 consecutive bytes (w0 = bytes 0-3, w1 = 4-7) biased by `bias` -> 8 f16
 * (byte - bias_off) * d */
__device__ static inline half8_t bytes_to_half8(u32 w0, u32 w1, half2_t off, half2_t d2)
{
	half2_t a = (magic2(w0, 0x04010400u) - off) * d2;
	half2_t b = (magic2(w0, 0x04030402u) - off) * d2;
	half2_t c = (magic2(w1, 0x04010400u) - off) * d2;
	half2_t e = (magic2(w1, 0x04030402u) - off) * d2;
	half8_t r;
	r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
	r[4] = c[0]; r[5] = c[1]; r[6] = e[0]; r[7] = e[1];
	return r;
}

/*
 * One lane's raw share of block b of a weight row (see the layout note at
 * the top); ODD = b & 1, which fixes the block's alignment: Q8_0 blocks
 * start at 34b, Q4_0 at 18b, both 4-byte aligned for even b and 2 bytes off
 * for odd b.  Every load stays inside the row: an even block is never the
 * last of a row (rows hold an even number of blocks).
 */
template <int WT, int ODD> struct bsrc;

template <int ODD> struct bsrc<1, ODD> { /* Q8_0 */
	static constexpr int BB = 34;
	u32 q0[3], q1[3], sc;
	__device__ inline void load(const uint8_t *blk, int h)
	{
		if (ODD) { /* quants 8h.. at blk + 2 + 8h, aligned; scale high half of blk - 2 */
			const u32 *a = (const u32 *)(blk + 2 + 8 * h);
			q0[0] = a[0]; q0[1] = a[1];
			q1[0] = a[4]; q1[1] = a[5];
			sc = *(const u32 *)(blk - 2) >> 16;
		} else { /* window at blk + 8h, quants 2 bytes in */
			const u32 *a = (const u32 *)(blk + 8 * h);
			q0[0] = a[0]; q0[1] = a[1]; q0[2] = a[2];
			q1[0] = a[4]; q1[1] = a[5]; q1[2] = a[6];
			sc = *(const u32 *)blk & 0xffffu;
		}
	}
	__device__ inline void operands(half8_t &k0, half8_t &k1) const
	{
		u32 a0, a1, b0, b1;
		if (ODD) {
			a0 = q0[0]; a1 = q0[1]; b0 = q1[0]; b1 = q1[1];
		} else {
			a0 = __builtin_amdgcn_alignbit(q0[1], q0[0], 16);
			a1 = __builtin_amdgcn_alignbit(q0[2], q0[1], 16);
			b0 = __builtin_amdgcn_alignbit(q1[1], q1[0], 16);
			b1 = __builtin_amdgcn_alignbit(q1[2], q1[1], 16);
		}
		const _Float16 d = __builtin_bit_cast(_Float16, (unsigned short)sc);
		const half2_t d2 = {d, d};
		const half2_t off = {(_Float16)1152.0f, (_Float16)1152.0f}; /* 1024 + 128 */
		k0 = bytes_to_half8(a0 ^ 0x80808080u, a1 ^ 0x80808080u, off, d2);
		k1 = bytes_to_half8(b0 ^ 0x80808080u, b1 ^ 0x80808080u, off, d2);
	}
};

template <int ODD> struct bsrc<2, ODD> { /* Q4_0 */
	static constexpr int BB = 18;
	u32 q[3], sc;
	__device__ inline void load(const uint8_t *blk, int h)
	{
		if (ODD) { /* packed bytes 8h.. at blk + 2 + 8h, aligned */
			const u32 *a = (const u32 *)(blk + 2 + 8 * h);
			q[0] = a[0]; q[1] = a[1];
			sc = *(const u32 *)(blk - 2) >> 16;
		} else {
			const u32 *a = (const u32 *)(blk + 8 * h);
			q[0] = a[0]; q[1] = a[1]; q[2] = a[2];
			sc = *(const u32 *)blk & 0xffffu;
		}
	}
	__device__ inline void operands(half8_t &k0, half8_t &k1) const
	{
		u32 w0, w1;
		if (ODD) {
			w0 = q[0]; w1 = q[1];
		} else {
			w0 = __builtin_amdgcn_alignbit(q[1], q[0], 16);
			w1 = __builtin_amdgcn_alignbit(q[2], q[1], 16);
		}
		const _Float16 d = __builtin_bit_cast(_Float16, (unsigned short)sc);
		const half2_t d2 = {d, d};
		const half2_t off = {(_Float16)1032.0f, (_Float16)1032.0f}; /* 1024 + 8 */
		k0 = bytes_to_half8(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, off, d2);
		k1 = bytes_to_half8((w0 >> 4) & 0x0f0f0f0fu, (w1 >> 4) & 0x0f0f0f0fu, off, d2);
	}
};

/* the raw weights of one pipeline step: blocks 2s (even) and 2s+1 (odd) of
 * NG row groups of 32 rows */
template <int WT, int NG> struct bstep {
	bsrc<WT, 0> ev[NG];
	bsrc<WT, 1> od[NG];
	__device__ inline void load(const uint8_t *const (&row)[NG], int s, int h)
	{
		constexpr int BB = bsrc<WT, 0>::BB;
#pragma unroll
		for (int g = 0; g < NG; g++) {
			ev[g].load(row[g] + (size_t)(2 * s) * BB, h);
			od[g].load(row[g] + (size_t)(2 * s + 1) * BB, h);
		}
	}
};

/* ---------------------------------------------------------------------- */
/* the MFMA step shared by both GEMMs                                      */
/* ---------------------------------------------------------------------- */

/* acc[mb][g] += A[mb-th 32 rows][64 k of this step] . B_g, A from LDS */
template <int WT, int NG>
__device__ static inline void mfma_step(const _Float16 *sa, const bstep<WT, NG> &B,
					floatx16 (&acc)[2][NG], int lane)
{
	const int h = lane >> 5, r = lane & 31;
#pragma unroll
	for (int bb = 0; bb < 2; bb++) {
		half8_t bk[NG][2];
#pragma unroll
		for (int g = 0; g < NG; g++) {
			if (bb == 0)
				B.ev[g].operands(bk[g][0], bk[g][1]);
			else
				B.od[g].operands(bk[g][0], bk[g][1]);
		}
#pragma unroll
		for (int kh = 0; kh < 2; kh++) {
#pragma unroll
			for (int mb = 0; mb < 2; mb++) {
				const half8_t a = *(const half8_t *)(sa + (mb * 32 + r) * PF_LDA +
								     bb * 32 + kh * 16 + 8 * h);
#pragma unroll
				for (int g = 0; g < NG; g++)
					acc[mb][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
						a, bk[g][kh], acc[mb][g], 0, 0, 0);
			}
		}
	}
}

/* ---------------------------------------------------------------------- */
/* activation tiles                                                        */
/* ---------------------------------------------------------------------- */

/* gate/up: thread -> tile row tid/4, 16 k at 16*(tid%4) of the step, from
 * the fp32 token row of the pair (zeros for padding) */
struct xtile {
	float4 v[4];
	__device__ inline void load(const float *src, int s)
	{
		if (!src) {
#pragma unroll
			for (int i = 0; i < 4; i++)
				v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
			return;
		}
		const float4 *p = (const float4 *)(src + (size_t)s * PF_KB);
#pragma unroll
		for (int i = 0; i < 4; i++)
			v[i] = p[i];
	}
	__device__ inline void store(_Float16 *dst) const
	{
		half8_t a, b;
		a[0] = (_Float16)v[0].x; a[1] = (_Float16)v[0].y; a[2] = (_Float16)v[0].z;
		a[3] = (_Float16)v[0].w; a[4] = (_Float16)v[1].x; a[5] = (_Float16)v[1].y;
		a[6] = (_Float16)v[1].z; a[7] = (_Float16)v[1].w;
		b[0] = (_Float16)v[2].x; b[1] = (_Float16)v[2].y; b[2] = (_Float16)v[2].z;
		b[3] = (_Float16)v[2].w; b[4] = (_Float16)v[3].x; b[5] = (_Float16)v[3].y;
		b[6] = (_Float16)v[3].z; b[7] = (_Float16)v[3].w;
		*(half8_t *)dst = a;
		*(half8_t *)(dst + 8) = b;
	}
};

/* down: the same 64 x 64 tile of h, already f16 */
struct htile {
	half8_t v[2];
	__device__ inline void load(const _Float16 *src, int s)
	{
		const half8_t *p = (const half8_t *)(src + (size_t)s * PF_KB);
		v[0] = p[0];
		v[1] = p[1];
	}
	__device__ inline void store(_Float16 *dst) const
	{
		*(half8_t *)dst = v[0];
		*(half8_t *)(dst + 8) = v[1];
	}
};

/*
 * The K loop: activation tile double-buffered in LDS, weights of the next
 * step loaded into registers while this step's MFMAs run.
 */
template <int WT, int NG, typename ATile, typename ASrc>
__device__ static inline void gemm_loop(_Float16 (*sa)[PF_MT * PF_LDA], ASrc asrc,
					const uint8_t *const (&brow)[NG], int nsteps,
					floatx16 (&acc)[2][NG])
{
	const int lane = threadIdx.x & 63, h = lane >> 5;
	_Float16 *adst0 = sa[0] + (threadIdx.x >> 2) * PF_LDA + 16 * (threadIdx.x & 3);
	_Float16 *adst1 = sa[1] + (threadIdx.x >> 2) * PF_LDA + 16 * (threadIdx.x & 3);
	ATile at;
	bstep<WT, NG> b0, b1;
	at.load(asrc, 0);
	b0.load(brow, 0, h);
	at.store(adst0);
	__syncthreads();
	for (int s = 0; s < nsteps; s += 2) {
		const bool more1 = s + 1 < nsteps;
		if (more1) {
			at.load(asrc, s + 1);
			b1.load(brow, s + 1, h);
		}
		mfma_step<WT, NG>(sa[0], b0, acc, lane);
		if (more1)
			at.store(adst1);
		__syncthreads();
		if (!more1)
			break;
		const bool more2 = s + 2 < nsteps;
		if (more2) {
			at.load(asrc, s + 2);
			b0.load(brow, s + 2, h);
		}
		mfma_step<WT, NG>(sa[1], b1, acc, lane);
		if (more2)
			at.store(adst0);
		__syncthreads();
	}
}

/* ---------------------------------------------------------------------- */
/* GEMM kernels                                                            */
/* ---------------------------------------------------------------------- */

template <int WT>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_gateup(
	const float *__restrict__ x, const uint8_t *__restrict__ gate,
	const uint8_t *__restrict__ up, size_t gu_stride, const int *__restrict__ rows,
	const int *__restrict__ tile_e, int K, int E, int EI, _Float16 *__restrict__ h)
{
	__shared__ __attribute__((aligned(16))) _Float16 sa[2][PF_MT * PF_LDA];
	const int tile = blockIdx.y;
	const int e = tile_e[tile];
	if (e < 0)
		return;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const size_t rb = (size_t)(E / MOE_QK) * bsrc<WT, 0>::BB;
	const int col = blockIdx.x * PF_GU_COLS + wave * 32 + (lane & 31);
	const uint8_t *const brow[2] = {gate + (size_t)e * gu_stride + (size_t)col * rb,
					up + (size_t)e * gu_stride + (size_t)col * rb};
	const int p = rows[tile * PF_MT + (threadIdx.x >> 2)];
	const float *asrc = p >= 0 ? x + (size_t)(p / K) * E + 16 * (threadIdx.x & 3) : nullptr;

	floatx16 acc[2][2];
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	gemm_loop<WT, 2, xtile>(sa, asrc, brow, E / PF_KB, acc);

	const int hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int row = tile * PF_MT + mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4);
			const float g = acc[mb][0][j], u = acc[mb][1][j];
			h[(size_t)row * EI + col] = (_Float16)((g / (1.0f + moe_expf(-g))) * u);
		}
}

template <int WT>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_down(
	const _Float16 *__restrict__ h, const uint8_t *__restrict__ down, size_t dn_stride,
	const int *__restrict__ rows, const int *__restrict__ tile_e, int E, int EI,
	float *__restrict__ ypart)
{
	__shared__ __attribute__((aligned(16))) _Float16 sa[2][PF_MT * PF_LDA];
	__shared__ int srow[PF_MT];
	const int tile = blockIdx.y;
	const int e = tile_e[tile];
	if (e < 0)
		return;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	if (threadIdx.x < PF_MT)
		srow[threadIdx.x] = rows[tile * PF_MT + threadIdx.x];
	const size_t rb = (size_t)(EI / MOE_QK) * bsrc<WT, 0>::BB;
	const int col0 = blockIdx.x * PF_DN_COLS + wave * 64 + (lane & 31);
	const uint8_t *base = down + (size_t)e * dn_stride;
	const uint8_t *const brow[2] = {base + (size_t)col0 * rb, base + (size_t)(col0 + 32) * rb};
	const _Float16 *asrc = h + (size_t)(tile * PF_MT + (threadIdx.x >> 2)) * EI +
			       16 * (threadIdx.x & 3);

	floatx16 acc[2][2];
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	gemm_loop<WT, 2, htile>(sa, asrc, brow, EI / PF_KB, acc); /* syncs srow too */

	const int hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int pr = srow[mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4)];
			if (pr < 0)
				continue;
#pragma unroll
			for (int g = 0; g < 2; g++)
				ypart[(size_t)pr * E + col0 + 32 * g] = acc[mb][g][j];
		}
}

/* ---------------------------------------------------------------------- */
/* host                                                                    */
/* ---------------------------------------------------------------------- */

extern "C" int moe_prefill_supported(int wtype, size_t E, size_t EI, size_t NE)
{
	return (wtype == 1 || wtype == 2) && NE <= MOE_MAX_NE && E % PF_DN_COLS == 0 &&
	       EI % PF_GU_COLS == 0 && E % PF_KB == 0 && EI % PF_KB == 0;
}

extern "C" int moe_prefill_max_tiles(size_t P, size_t NE)
{
	size_t t = (P + PF_MT - 1) / PF_MT + (NE < P ? NE : P);
	return (int)t;
}

extern "C" int moe_prefill_tile_rows(void)
{
	return PF_MT;
}

extern "C" int moe_launch_prefill(int wtype, const float *x, const uint8_t *gate,
				  const uint8_t *up, const uint8_t *down, size_t gu_stride,
				  size_t dn_stride, const uint32_t *ids, int *rows, int *tile_e,
				  void *h16, float *ypart, int T, int K, int E, int EI, int NE,
				  void *stream)
{
	if (!moe_prefill_supported(wtype, (size_t)E, (size_t)EI, (size_t)NE))
		return (int)hipErrorInvalidValue;
	hipStream_t s = (hipStream_t)stream;
	const int P = T * K;
	const int Tmax = moe_prefill_max_tiles((size_t)P, (size_t)NE);
	hipLaunchKernelGGL(k_moe_sort, dim3(1), dim3(SORT_THREADS), 0, s, ids, P, NE, Tmax, rows,
			   tile_e);
	_Float16 *hh = (_Float16 *)h16;
	if (wtype == 1) {
		hipLaunchKernelGGL(k_pf_gateup<1>, dim3(EI / PF_GU_COLS, Tmax), dim3(PF_THREADS), 0,
				   s, x, gate, up, gu_stride, rows, tile_e, K, E, EI, hh);
		hipLaunchKernelGGL(k_pf_down<1>, dim3(E / PF_DN_COLS, Tmax), dim3(PF_THREADS), 0, s,
				   hh, down, dn_stride, rows, tile_e, E, EI, ypart);
	} else {
		hipLaunchKernelGGL(k_pf_gateup<2>, dim3(EI / PF_GU_COLS, Tmax), dim3(PF_THREADS), 0,
				   s, x, gate, up, gu_stride, rows, tile_e, K, E, EI, hh);
		hipLaunchKernelGGL(k_pf_down<2>, dim3(E / PF_DN_COLS, Tmax), dim3(PF_THREADS), 0, s,
				   hh, down, dn_stride, rows, tile_e, E, EI, ypart);
	}
	return (int)hipGetLastError();
}
