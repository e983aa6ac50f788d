/*
 * Prefill-sized MoE FFN layer: tokens sorted by expert, then grouped GEMMs
 * on the f16 matrix cores.
 *
 *   k_moe_sort     counting sort of the T*K (token, slot) pairs by
 *                  expert into m-tiles of MT rows (the tail of each
 *                  expert's last tile is padding, row id -1), and the tile
 *                  table tile -> expert.  MT = 64, or 32 when the experts
 *                  average fewer than 32 pairs (the MFMAs of a tile's
 *                  second 32 rows would be padding).  Inside an expert
 *                  the pairs land in the order the LDS atomics give; a
 *                  row's products do not depend on its place in the tile.
 *   k_pf_gateup    per (m-tile, 256 h columns): G = X Wg^T and U = X Wu^T
 *                  over d_model, h = silu(G) * U  (nn.c:460-478), stored f16
 *                  in sorted row order.  X is the f16 copy of the tokens the
 *                  router kernel writes.
 *   k_pf_down      per (m-tile, 512 output columns, K-split): Y = H Wd^T
 *                  (the down matrices are stored as panels: panel c holds
 *                  block c of every row, so a stage reads two contiguous
 *                  runs of 512 blocks)
 *                  over d_ff (or one of S consecutive parts of it, when the
 *                  tiles alone leave the CUs idle), written fp32 to
 *                  ypart[pair][split][E]; k_combine then adds the splits in
 *                  order and the slots of each token in order,
 *                  out += y / (1/w)  (olmoe.c:401-403).
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

#define PF_MT_MAX 64        /* rows (pairs) per m-tile: 32 or 64 */
#define PF_KB 64            /* k per pipeline step: two blocks */
#define SORT_THREADS 1024

/* ---------------------------------------------------------------------- */
/* sort                                                                    */
/* ---------------------------------------------------------------------- */

/*
 * One workgroup.  Counts per expert, tiles per expert (exclusive scan), the
 * tile table, padding rows (-1), then every pair's row: toff[e] * MT + a
 * slot taken with an LDS atomic.  The order of the pairs inside an expert
 * may differ between calls, but the results do not: every output row of
 * the GEMMs depends only on its own activation row (the row's MFMA sums do
 * not involve the other rows of its tile).  rows[] gets Tmax*MT entries
 * and tile_e[] Tmax + 1 entries (-1 past the last tile, then the number of
 * tiles in use), all rewritten on every call.
 */
#define SORT_MAX_TILES 8704 /* Tmax for T*K up to 2^19 pairs and NE <= 256 */

/* ids a sort thread takes per round: one 16-byte load (with 16 a thread,
 * the 256 threads that had ids did all the counting and placing: 6.9 us a
 * sort at OLMoE T = 512, 2.8 of them counting) */
#define SORT_IPT 4

/* ids p0 .. p0 + SORT_IPT - 1 (~0 past P) */
__device__ static inline void sort_ids(const u32 *ids, int p0, int P, u32 (&v)[SORT_IPT])
{
	if (p0 + SORT_IPT <= P && ((uintptr_t)(ids + p0) & 15) == 0) {
		const uint4 q = *(const uint4 *)(ids + p0);
		v[0] = q.x;
		v[1] = q.y;
		v[2] = q.z;
		v[3] = q.w;
	} else {
#pragma unroll
		for (int k = 0; k < SORT_IPT; k++)
			v[k] = p0 + k < P ? ids[p0 + k] : 0xffffffffu;
	}
}

template <int MT>
__global__ __launch_bounds__(SORT_THREADS) void k_moe_sort(const u32 *__restrict__ ids, int P,
							   int NE, int Tmax,
							   int *__restrict__ rows,
							   int *__restrict__ tile_e)
{
	__shared__ int cnt[MOE_MAX_NE], toff[MOE_MAX_NE + 1], fill[MOE_MAX_NE];
	__shared__ short stile[SORT_MAX_TILES];
	const int tid = threadIdx.x;

	for (int i = tid; i < NE; i += SORT_THREADS) {
		cnt[i] = 0;
		fill[i] = 0;
	}
	__syncthreads();
	/* counts: SORT_IPT ids per thread and round, loaded together; the
	 * first round's ids stay in registers for the placement below */
	u32 v0[SORT_IPT];
	for (int p0 = SORT_IPT * tid; p0 < P; p0 += SORT_IPT * SORT_THREADS) {
		u32 v[SORT_IPT];
		sort_ids(ids, p0, P, v);
#pragma unroll
		for (int k = 0; k < SORT_IPT; k++) {
			if (p0 == SORT_IPT * tid)
				v0[k] = v[k];
			if (v[k] < (u32)NE) /* always, for ids from the top-k kernel */
				atomicAdd(&cnt[v[k]], 1);
		}
	}
	__syncthreads();
	if (tid < WAVE) { /* exclusive scan of tiles per expert, 4 experts per lane */
		const int lane = tid;
		int t4[4], s = 0;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int ex = 4 * lane + i;
			t4[i] = ex < NE ? (cnt[ex] + MT - 1) / MT : 0;
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
	if (tid == 0)
		tile_e[Tmax] = ntiles;
	/* tile table: the expert of each tile (largest e with toff[e] <= tile) */
	for (int tl = tid; tl < Tmax; tl += SORT_THREADS) {
		int ex = -1;
		if (tl < ntiles) {
			int lo = 0, hi = NE - 1;
			while (lo < hi) {
				const int mid = (lo + hi + 1) >> 1;
				if (toff[mid] <= tl)
					lo = mid;
				else
					hi = mid - 1;
			}
			ex = lo;
		}
		stile[tl] = (short)ex;
		tile_e[tl] = ex;
	}
	__syncthreads();
	/* padding rows */
	for (int i = tid; i < Tmax * MT; i += SORT_THREADS) {
		const int ex = stile[i / MT];
		if (ex < 0 || i - toff[ex] * MT >= cnt[ex])
			rows[i] = -1;
	}
	/* every pair's row */
	for (int p0 = SORT_IPT * tid; p0 < P; p0 += SORT_IPT * SORT_THREADS) {
		u32 v[SORT_IPT];
		if (p0 == SORT_IPT * tid) {
#pragma unroll
			for (int k = 0; k < SORT_IPT; k++)
				v[k] = v0[k];
		} else {
			sort_ids(ids, p0, P, v);
		}
#pragma unroll
		for (int k = 0; k < SORT_IPT; k++)
			if (v[k] < (u32)NE)
				rows[toff[v[k]] * MT + atomicAdd(&fill[v[k]], 1)] = p0 + k;
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

/* ---------------------------------------------------------------------- */
/* the grouped GEMMs                                                       */
/* ---------------------------------------------------------------------- */

/*
 * A workgroup of 8 waves computes a 64-row m-tile against 512 weight rows
 * (2 groups of 32 rows per wave) over the whole K: Q8_0 one per CU with a
 * 3-stage ring, Q4_0 two per CU with a 2-stage ring, so that one
 * dequantizes while the other's MFMAs run.  Each K-step
 * (PF_KB = 64: two GGML blocks per row) goes through an LDS ring of NS
 * stages filled by LDS-DMA loads (global_load_lds: no registers, so
 * NS - 1 stages stay in flight):
 *   B part: the raw blocks of the 512 rows, [row][16-byte chunks];
 *   A part: 64 rows x 64 f16 activations, 16-byte chunk c of row r at slot
 *           8r + (c ^ (r & 7)) (conflict-free MFMA operand reads).
 * The loads are issued from inline assembly, so the compiler neither tracks
 * nor waits for them; the K loop waits itself: vmcnt counts this wave's
 * loads and retires them in issue order, and a barrier then makes every
 * wave's part of the stage visible.
 */
#define PF_WAVES 8
#define PF_BROWS 512 /* weight rows per workgroup */

template <int WT, int AL = 1> struct pf_geo { /* AL: A loads per thread (64 rows each) */
	static constexpr int BB = WT == 1 ? 34 : 18;    /* block bytes */
	static constexpr int RBS = 2 * BB;               /* bytes of a row per stage */
	/* 16-byte chunks loaded per row and stage (LDS-DMA writes one 16-byte
	 * slot per lane): they cover the RBS bytes and run up to 12 bytes into
	 * the next stage's (the weights allocation carries slack for the last
	 * row) */
	static constexpr int CH = 16;                    /* chunk bytes */
	static constexpr int NCH = (RBS + CH - 1) / CH;
	static constexpr int RBL = CH * NCH;             /* LDS bytes per row */
	static constexpr int JB = PF_BROWS * NCH / (PF_WAVES * WAVE); /* B loads per wave */
	static constexpr int BSZ = PF_BROWS * RBL;       /* B bytes per stage */
	static constexpr int ASZ = 64 * AL * PF_KB * 2; /* A bytes per stage */
	static constexpr int SSZ = BSZ + ASZ;
	static constexpr int LOADS = JB + AL;            /* loads per wave per stage */
};


/* acc[mb][g] += A[mb-th 32 rows] . B_g over one stage, mb < MB.  Every LDS
 * read of the stage is issued first, so the stage waits for LDS once, not
 * once per operand. */
template <int WT, int MB>
__device__ static inline void pf_stage_mfma(const uint8_t *sb, const _Float16 *sa,
					    const int (&brow)[2], floatx16 (&acc)[MB < 2 ? 2 : MB][2],
					    int lane)
{
	typedef pf_geo<WT> GG;
	const int h = lane >> 5, r = lane & 31;
	bsrc<WT, 0> ev[2];
	bsrc<WT, 1> od[2];
	half8_t a[2][2][MB]; /* [block][k-half][mb] */
#pragma unroll
	for (int g = 0; g < 2; g++) {
		const uint8_t *row = sb + brow[g] * GG::RBS;
		ev[g].load(row, h);
		od[g].load(row + GG::BB, h);
	}
#pragma unroll
	for (int bb = 0; bb < 2; bb++)
#pragma unroll
		for (int kh = 0; kh < 2; kh++)
#pragma unroll
			for (int mb = 0; mb < MB; mb++) {
				const int ar = mb * 32 + r, c = bb * 4 + kh * 2 + h;
				a[bb][kh][mb] = *(const half8_t *)(sa + 8 * (ar * 8 + (c ^ (ar & 7))));
			}
#pragma unroll
	for (int bb = 0; bb < 2; bb++) {
		half8_t bk[2][2]; /* [group][k-half] */
#pragma unroll
		for (int g = 0; g < 2; g++) {
			if (bb == 0)
				ev[g].operands(bk[g][0], bk[g][1]);
			else
				od[g].operands(bk[g][0], bk[g][1]);
		}
#pragma unroll
		for (int kh = 0; kh < 2; kh++)
#pragma unroll
			for (int mb = 0; mb < MB; mb++)
#pragma unroll
				for (int g = 0; g < 2; g++)
					acc[mb][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
						a[bb][kh][mb], bk[g][kh], acc[mb][g], 0, 0, 0);
	}
}

/* The same for a stage of two down panels: LDS holds rows n0 .. n0+511 of
 * panel 2s, then of panel 2s+1 (PF_BROWS blocks each, unpadded).  The lane's
 * column pair is rows n (even: 4-byte aligned blocks) and n+1 (odd: 2 bytes
 * off), so each group reads blocks of one alignment. */
template <int WT, int MB>
__device__ static inline void pf_stage_mfma_panel(const uint8_t *sb, const _Float16 *sa, int n,
						  floatx16 (&acc)[MB < 2 ? 2 : MB][2], int lane)
{
	typedef pf_geo<WT> GG;
	constexpr int RUN = PF_BROWS * GG::BB;
	const int h = lane >> 5, r = lane & 31;
	bsrc<WT, 0> ev[2]; /* [panel]: row n */
	bsrc<WT, 1> od[2]; /* [panel]: row n + 1 */
#pragma unroll
	for (int pp = 0; pp < 2; pp++) {
		ev[pp].load(sb + pp * RUN + n * GG::BB, h);
		od[pp].load(sb + pp * RUN + (n + 1) * GG::BB, h);
	}
	half8_t a[2][2][MB]; /* [block][k-half][mb] */
#pragma unroll
	for (int bb = 0; bb < 2; bb++)
#pragma unroll
		for (int kh = 0; kh < 2; kh++)
#pragma unroll
			for (int mb = 0; mb < MB; mb++) {
				const int ar = mb * 32 + r, c = bb * 4 + kh * 2 + h;
				a[bb][kh][mb] = *(const half8_t *)(sa + 8 * (ar * 8 + (c ^ (ar & 7))));
			}
#pragma unroll
	for (int bb = 0; bb < 2; bb++) {
		half8_t bk[2][2]; /* [group][k-half] */
		ev[bb].operands(bk[0][0], bk[0][1]);
		od[bb].operands(bk[1][0], bk[1][1]);
#pragma unroll
		for (int kh = 0; kh < 2; kh++)
#pragma unroll
			for (int mb = 0; mb < MB; mb++)
#pragma unroll
				for (int g = 0; g < 2; g++)
					acc[mb][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
						a[bb][kh][mb], bk[g][kh], acc[mb][g], 0, 0, 0);
	}
}

/*
 * The K loop.  wbase: weights base (SGPR); woff[j]: this lane's byte offset
 * of load j of stage 0; abase/aoff the same for A.  Stage s adds s * wstep
 * (weights) and s * 128 (A) to the bases.  PANEL: the stage holds two down
 * panels (brow[0] = the lane's even row) instead of [row][chunk] rows.
 */
template <int WT, int PANEL, int NS, int MB, int AL = 1>
__device__ static inline void pf_kloop(uint8_t *lds, const uint8_t *wbase, size_t wstep,
				       const u32 (&woff)[pf_geo<WT>::JB], const uint8_t *abase,
				       const u32 (&aoff)[AL], const int (&brow)[2], int nsteps,
				       floatx16 (&acc)[MB < 2 ? 2 : MB][2])
{
	typedef pf_geo<WT, AL> GG;
	constexpr bool HALF_A = MB == 1 && AL == 1 && NS == 2;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const u32 l0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
	auto issue = [&](int s) {
		const u32 st = l0 + (u32)((s % NS) * GG::SSZ);
		const uint8_t *wb = wbase + (size_t)s * wstep;
#pragma unroll
		for (int j = 0; j < GG::JB; j++)
			dma_dwordx4(wb, woff[j], st + (u32)((wave * GG::JB + j) * WAVE * GG::CH));
		/* lanes of padding rows all read the same 16 bytes; a 32-row
		 * tile's waves 4-7 would load only rows 32-63, which no MFMA
		 * reads, so a 2-stage ring (which waits for all of a wave's
		 * loads) skips them: Mixtral T=64 217.1 -> 213.0 us, T=16 209.3
		 * -> 204.9 us.  In the 4-stage ring the waves' uneven waits cost
		 * more than the loads (OLMoE T=512 155.2 -> 157.3 us). */
#pragma unroll
		for (int a = 0; a < AL; a++)
			if (!HALF_A || wave < 4)
				dma_dwordx4(abase + (size_t)s * 128, aoff[a],
					    st + GG::BSZ + (u32)(a * 8192 + wave * 1024));
	};
#pragma unroll
	for (int s = 0; s < NS - 1; s++)
		if (s < nsteps)
			issue(s);
	for (int s = 0; s < nsteps; s++) {
		if (s + NS - 2 < nsteps)
			wait_vm<(NS - 2) * GG::LOADS>();
		else
			wait_vm<0>();
		__syncthreads(); /* stage s landed for every wave; stage s-1 is free */
		if (s + NS - 1 < nsteps)
			issue(s + NS - 1);
		const uint8_t *sb = lds + (s % NS) * GG::SSZ;
		__builtin_amdgcn_s_setprio(1);
		if (PANEL)
			pf_stage_mfma_panel<WT, MB>(sb, (const _Float16 *)(sb + GG::BSZ), brow[0],
						    acc, lane);
		else
			pf_stage_mfma<WT, MB>(sb, (const _Float16 *)(sb + GG::BSZ), brow, acc, lane);
		__builtin_amdgcn_s_setprio(0);
	}
}

/*
 * Work order of a GEMM grid (nb column blocks fastest, then tiles): the
 * workgroups are dealt round-robin over the 8 XCDs, so workgroup class
 * id % 8 shares one L2; each class takes a contiguous run of the
 * nb * ntiles items in use, so an expert's m-tiles run side by side on one
 * L2 and read its weights once from HBM.  Returns false for a workgroup
 * without an item.
 */
__device__ static inline bool pf_item(int ntiles, int &tile, int &nb)
{
	const int NB = (int)gridDim.x, G = NB * (int)gridDim.y;
	const int id = (int)blockIdx.x + NB * (int)blockIdx.y, U = NB * ntiles;
	int L = id;
	if (G % 8 == 0) {
		const int share = (U + 7) / 8;
		if (id / 8 >= share)
			return false;
		L = (id % 8) * share + id / 8;
	}
	if (L >= U)
		return false;
	tile = L / NB;
	nb = L % NB;
	return true;
}

/* this lane's A chunk of a stage (slot -> row, chunk) */
template <int WT> struct pf_lanes {
	int arow, achunk;
	__device__ inline pf_lanes()
	{
		const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
		const int slot = wave * WAVE + lane;
		arow = slot >> 3;
		achunk = (slot & 7) ^ (arow & 7);
	}
};

template <int WT, int NS, int MB>
__global__ __launch_bounds__(PF_WAVES * WAVE) void k_pf_gateup(
	const _Float16 *__restrict__ xh, const uint8_t *__restrict__ gate, size_t up_off,
	size_t gu_stride, const int *__restrict__ rows, const int *__restrict__ tile_e, int K,
	int E, int EI, _Float16 *__restrict__ h)
{
	typedef pf_geo<WT> GG;
	__shared__ __attribute__((aligned(16))) uint8_t lds[NS * GG::SSZ];
	int tile, nb;
	if (!pf_item(tile_e[gridDim.y], tile, nb))
		return;
	const int e = tile_e[tile];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int n0 = nb * (PF_BROWS / 2);
	const size_t rb = (size_t)(E / MOE_QK) * GG::BB;
	pf_lanes<WT> L;
	/* weight rows 0..255: gate rows n0.., 256..511: up rows n0.. (offsets
	 * from the gate base; up = gate + up_off).  A stage is piece s of every
	 * row: with the weights in MOE_GU_GROUP-row groups, one contiguous run
	 * of CPG 16-byte chunks per group (8 gate, then 8 up groups), landing
	 * as rows of RBS bytes; the spare lanes of the last loads reload the
	 * first chunk into LDS past the rows. */
	constexpr int CPG = MOE_GU_GROUP * GG::RBS / GG::CH;
	static_assert(MOE_GU_GROUP * GG::RBS % GG::CH == 0 && 16 * CPG <= GG::JB * PF_WAVES * WAVE,
		      "a stage's group runs fit the loads");
	u32 woff[GG::JB];
#pragma unroll
	for (int j = 0; j < GG::JB; j++) {
		const int f = (wave * GG::JB + j) * WAVE + lane, lg = f / CPG; /* its LDS slot */
		const size_t o = f < 16 * CPG
					 ? (lg < 8 ? 0 : up_off) + (size_t)e * gu_stride +
						   (size_t)(n0 + MOE_GU_GROUP * (lg & 7)) * rb +
						   (size_t)GG::CH * (f % CPG)
					 : (size_t)e * gu_stride + (size_t)n0 * rb;
		woff[j] = (u32)o;
	}
	constexpr int MT = 32 * MB;
	const int p = L.arow < MT ? rows[tile * MT + L.arow] : -1;
	/* padding rows (and the stage's rows past MT): one shared 16-byte chunk
	 * instead of a row each */
	const u32 aoff[1] = {p >= 0 ? (u32)((size_t)(p / K) * E * 2 + 16 * L.achunk) : 0u};
	const int brow[2] = {wave * 32 + (lane & 31), 256 + wave * 32 + (lane & 31)};

	floatx16 acc[2][2];
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	pf_kloop<WT, 0, NS, MB>(lds, gate, MOE_GU_GROUP * GG::RBS, woff, (const uint8_t *)xh, aoff,
				brow, E / PF_KB, acc);

	const int col = n0 + wave * 32 + (lane & 31), hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < MB; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int row = tile * MT + mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4);
			const float g = acc[mb][0][j], u = acc[mb][1][j];
			h[(size_t)row * EI + col] = (_Float16)((g / (1.0f + moe_expf(-g))) * u);
		}
}

template <int WT, int NS, int MB>
__global__ __launch_bounds__(PF_WAVES * WAVE) void k_pf_down(
	const _Float16 *__restrict__ h, const uint8_t *__restrict__ down, size_t dn_stride,
	const int *__restrict__ rows, const int *__restrict__ tile_e, int E, int EI,
	float *__restrict__ ypart)
{
	typedef pf_geo<WT> GG;
	__shared__ __attribute__((aligned(16))) uint8_t lds[NS * GG::SSZ];
	constexpr int MT = 32 * MB;
	__shared__ int srow[MT];
	int tile, nb;
	if (!pf_item(tile_e[gridDim.y], tile, nb))
		return;
	const int e = tile_e[tile];
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int S = gridDim.z, nst = EI / PF_KB;
	const int s0 = blockIdx.z * nst / S, s1 = (blockIdx.z + 1) * nst / S;
	if (threadIdx.x < MT)
		srow[threadIdx.x] = rows[tile * MT + threadIdx.x];
	const int n0 = nb * PF_BROWS;
	/* stage s = rows n0 .. n0+511 of panels 2s and 2s+1: two contiguous runs
	 * of RUN bytes, loaded as 16-byte chunks; chunks past them (the last
	 * wave's spare lanes) reload chunk 0 into unused LDS */
	const size_t RUN = (size_t)PF_BROWS * GG::BB, PANEL = (size_t)E * GG::BB;
	pf_lanes<WT> L;
	u32 woff[GG::JB];
#pragma unroll
	for (int j = 0; j < GG::JB; j++) {
		const size_t f = (size_t)((wave * GG::JB + j) * WAVE + lane) * GG::CH;
		woff[j] = (u32)((size_t)e * dn_stride +
				(f < 2 * RUN ? (f / RUN) * PANEL + (size_t)n0 * GG::BB + f % RUN
					     : (size_t)n0 * GG::BB));
	}
	const u32 aoff[1] = {L.arow < MT && rows[tile * MT + L.arow] >= 0
				     ? (u32)((size_t)(tile * MT + L.arow) * EI * 2 + 16 * L.achunk)
				     : 0u};
	/* MFMA column r of group g = output row wave*64 + 2r + g */
	const int brow[2] = {wave * 64 + 2 * (lane & 31), wave * 64 + 2 * (lane & 31) + 1};

	floatx16 acc[2][2];
#pragma unroll
	for (int mb = 0; mb < 2; mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	pf_kloop<WT, 1, NS, MB>(lds, down + (size_t)s0 * 2 * PANEL, 2 * PANEL, woff,
			(const uint8_t *)(h + (size_t)s0 * PF_KB), aoff, brow, s1 - s0,
			acc); /* syncs srow */

	const int hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < MB; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int pr = srow[mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4)];
			if (pr < 0)
				continue;
#pragma unroll
			for (int g = 0; g < 2; g++)
				ypart[((size_t)pr * S + blockIdx.z) * E + n0 + wave * 64 +
				      2 * (lane & 31) + g] = acc[mb][g][j];
		}
}

/* ---------------------------------------------------------------------- */
/* tiles of 32, 64 or 128 rows per expert                                  */
/* ---------------------------------------------------------------------- */

/*
 * With many pairs per expert (prefill), an expert of c pairs takes
 * floor(c / 128) tiles of 128 rows, and its remainder r one more tile: of
 * 128 rows if r > 64, of 64 if r > 32, of 32 if r > 0.  A 128-row tile
 * feeds each dequantised weight block to twice the MFMAs of a 64-row one
 * (the dequantisation is most of a K-step's VALU work), and the tails keep
 * the padding of light experts under 32 rows.  The tile list puts every
 * 128-row tile first, then the 64- and the 32-row tails, so the largest
 * items are dealt out first.
 *
 * tinfo[0] = tiles in use; tile i: tinfo[1 + 2i] = expert | rows/32 << 16,
 * tinfo[2 + 2i] = its first row.  rows[] holds each expert's pairs at its
 * first row on, padding -1 to the end of its last tile.  One workgroup;
 * every entry it names is rewritten on every call (graph-safe).
 */
__global__ __launch_bounds__(SORT_THREADS) void k_moe_sort_v(const u32 *__restrict__ ids, int P,
							     int NE, int Tmax,
							     int *__restrict__ rows,
							     int *__restrict__ tinfo)
{
	__shared__ int cnt[MOE_MAX_NE], fill[MOE_MAX_NE];
	__shared__ int rb[MOE_MAX_NE], p4[MOE_MAX_NE], p2[MOE_MAX_NE], p1[MOE_MAX_NE];
	__shared__ int s_tot[4]; /* rows, 128-, 64-, 32-row tiles */
	const int tid = threadIdx.x;
	for (int i = tid; i < NE; i += SORT_THREADS) {
		cnt[i] = 0;
		fill[i] = 0;
	}
	__syncthreads();
	u32 v0[SORT_IPT];
	for (int p0 = SORT_IPT * tid; p0 < P; p0 += SORT_IPT * SORT_THREADS) {
		u32 v[SORT_IPT];
		sort_ids(ids, p0, P, v);
#pragma unroll
		for (int k = 0; k < SORT_IPT; k++) {
			if (p0 == SORT_IPT * tid)
				v0[k] = v[k];
			if (v[k] < (u32)NE)
				atomicAdd(&cnt[v[k]], 1);
		}
	}
	__syncthreads();
	if (tid < WAVE) { /* exclusive scans over experts, 4 per lane */
		const int lane = tid;
		int r4[4], n4[4], t2[4], t1[4], sr = 0, s4 = 0, s2 = 0, s1 = 0;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int ex = 4 * lane + i;
			const int c = ex < NE ? cnt[ex] : 0;
			int n = c / 128;
			const int rem = c - 128 * n;
			int tail = 0;
			if (rem > 64)
				n++;
			else if (rem > 32)
				tail = 2;
			else if (rem > 0)
				tail = 1;
			n4[i] = n;
			t2[i] = tail == 2;
			t1[i] = tail == 1;
			r4[i] = 128 * n + 32 * tail;
			sr += r4[i];
			s4 += n4[i];
			s2 += t2[i];
			s1 += t1[i];
		}
		int ir = sr, i4 = s4, i2 = s2, i1 = s1;
#pragma unroll
		for (int d = 1; d < WAVE; d <<= 1) {
			const int a = __shfl_up(ir, d, WAVE), b = __shfl_up(i4, d, WAVE);
			const int c = __shfl_up(i2, d, WAVE), e = __shfl_up(i1, d, WAVE);
			if (lane >= d) {
				ir += a;
				i4 += b;
				i2 += c;
				i1 += e;
			}
		}
		int br = ir - sr, b4 = i4 - s4, b2 = i2 - s2, b1 = i1 - s1;
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const int ex = 4 * lane + i;
			if (ex < NE) {
				rb[ex] = br;
				p4[ex] = b4;
				p2[ex] = b2;
				p1[ex] = b1;
			}
			br += r4[i];
			b4 += n4[i];
			b2 += t2[i];
			b1 += t1[i];
		}
		if (lane == WAVE - 1) {
			s_tot[0] = ir;
			s_tot[1] = i4;
			s_tot[2] = i2;
			s_tot[3] = i1;
		}
	}
	__syncthreads();
	const int T4 = s_tot[1], T2 = s_tot[2], T1 = s_tot[3], ntiles = T4 + T2 + T1;
	if (tid == 0)
		tinfo[0] = ntiles;
	/* the tile list */
	for (int ex = tid; ex < NE; ex += SORT_THREADS) {
		const int c = cnt[ex];
		int n = c / 128;
		const int rem = c - 128 * n;
		int tail = 0;
		if (rem > 64)
			n++;
		else if (rem > 32)
			tail = 2;
		else if (rem > 0)
			tail = 1;
		for (int i = 0; i < n; i++) {
			tinfo[1 + 2 * (p4[ex] + i)] = ex | (4 << 16);
			tinfo[2 + 2 * (p4[ex] + i)] = rb[ex] + 128 * i;
		}
		if (tail) {
			const int tl = tail == 2 ? T4 + p2[ex] : T4 + T2 + p1[ex];
			tinfo[1 + 2 * tl] = ex | (tail << 16);
			tinfo[2 + 2 * tl] = rb[ex] + 128 * n;
		}
	}
	for (int tl = ntiles + tid; tl < Tmax; tl += SORT_THREADS) {
		tinfo[1 + 2 * tl] = -1;
		tinfo[2 + 2 * tl] = 0;
	}
	/* padding rows, then every pair's row */
	const int R = s_tot[0];
	for (int i = tid; i < R; i += SORT_THREADS)
		rows[i] = -1;
	__syncthreads();
	for (int p0 = SORT_IPT * tid; p0 < P; p0 += SORT_IPT * SORT_THREADS) {
		u32 v[SORT_IPT];
		if (p0 == SORT_IPT * tid) {
#pragma unroll
			for (int k = 0; k < SORT_IPT; k++)
				v[k] = v0[k];
		} else {
			sort_ids(ids, p0, P, v);
		}
#pragma unroll
		for (int k = 0; k < SORT_IPT; k++)
			if (v[k] < (u32)NE)
				rows[rb[v[k]] + atomicAdd(&fill[v[k]], 1)] = p0 + k;
	}
}

/* item of a variable-tile grid: in dispatch order, which is the tile list's
 * (the largest tiles first) with each tile's column blocks side by side;
 * consecutive workgroups land on different XCDs, so the 128-row tiles
 * spread over all of them */
__device__ static inline bool pf_item_v(int ntiles, int &tile, int &nb)
{
	const int NB = (int)gridDim.x, L = (int)blockIdx.x + NB * (int)blockIdx.y;
	if (L >= NB * ntiles)
		return false;
	tile = L / NB;
	nb = L % NB;
	return true;
}

/* this lane's A chunks: row arow of a stage, and row arow + 64 for tiles over 64 rows */
struct pf_lanes2 {
	int arow, achunk;
	__device__ inline pf_lanes2()
	{
		const int slot = threadIdx.x; /* 0 .. 511: rows 0 .. 63 */
		arow = slot >> 3;
		achunk = (slot & 7) ^ (arow & 7);
	}
};

/* one gate/up tile of 32 * MB rows starting at row r0 (expert e) */
template <int WT, int NS, int MB>
__device__ static void pf_gateup_tile(uint8_t *lds, const _Float16 *xh, const uint8_t *gate,
				      size_t up_off, size_t gu_stride, const int *rows, int K,
				      int E, int EI, _Float16 *h, int e, int r0, int nb)
{
	constexpr int AL = MB > 2 ? 2 : 1; /* 64-row A loads: tiles up to 64 rows need one */
	typedef pf_geo<WT, AL> GG;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int n0 = nb * (PF_BROWS / 2);
	const size_t rb = (size_t)(E / MOE_QK) * GG::BB;
	constexpr int CPG = MOE_GU_GROUP * GG::RBS / GG::CH;
	u32 woff[GG::JB];
#pragma unroll
	for (int j = 0; j < GG::JB; j++) {
		const int f = (wave * GG::JB + j) * WAVE + lane, lg = f / CPG;
		const size_t o = f < 16 * CPG
					 ? (lg < 8 ? 0 : up_off) + (size_t)e * gu_stride +
						   (size_t)(n0 + MOE_GU_GROUP * (lg & 7)) * rb +
						   (size_t)GG::CH * (f % CPG)
					 : (size_t)e * gu_stride + (size_t)n0 * rb;
		woff[j] = (u32)o;
	}
	constexpr int MT = 32 * MB;
	pf_lanes2 L;
	u32 aoff[AL];
#pragma unroll
	for (int a = 0; a < AL; a++) {
		const int ar = L.arow + 64 * a;
		const int p = ar < MT ? rows[r0 + ar] : -1;
		aoff[a] = p >= 0 ? (u32)((size_t)(p / K) * E * 2 + 16 * L.achunk) : 0u;
	}
	const int brow[2] = {wave * 32 + (lane & 31), 256 + wave * 32 + (lane & 31)};
	floatx16 acc[MB < 2 ? 2 : MB][2];
#pragma unroll
	for (int mb = 0; mb < (MB < 2 ? 2 : MB); mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	pf_kloop<WT, 0, NS, MB, AL>(lds, gate, MOE_GU_GROUP * GG::RBS, woff, (const uint8_t *)xh,
				   aoff, brow, E / PF_KB, acc);
	const int col = n0 + wave * 32 + (lane & 31), hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < MB; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int row = r0 + mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4);
			const float g = acc[mb][0][j], u = acc[mb][1][j];
			h[(size_t)row * EI + col] = (_Float16)((g / (1.0f + moe_expf(-g))) * u);
		}
}

/* k_pf_gateup over the tiles of k_moe_sort_v: one workgroup per CU (the
 * 128-row instance holds 4 x 2 accumulator tiles per wave) */
template <int WT, int NS>
__global__ __launch_bounds__(PF_WAVES * WAVE) void k_pf_gateup_v(
	const _Float16 *__restrict__ xh, const uint8_t *__restrict__ gate, size_t up_off,
	size_t gu_stride, const int *__restrict__ rows, const int *__restrict__ tinfo, int K,
	int E, int EI, _Float16 *__restrict__ h)
{
	__shared__ __attribute__((aligned(16))) uint8_t lds[NS * pf_geo<WT, 2>::SSZ];
	int tile, nb;
	if (!pf_item_v(tinfo[0], tile, nb))
		return;
	const int te = tinfo[1 + 2 * tile], e = te & 0xffff, mb = te >> 16, r0 = tinfo[2 + 2 * tile];
	if (mb == 4)
		pf_gateup_tile<WT, NS, 4>(lds, xh, gate, up_off, gu_stride, rows, K, E, EI, h, e, r0, nb);
	else if (mb == 2)
		pf_gateup_tile<WT, NS, 2>(lds, xh, gate, up_off, gu_stride, rows, K, E, EI, h, e, r0, nb);
	else
		pf_gateup_tile<WT, NS, 1>(lds, xh, gate, up_off, gu_stride, rows, K, E, EI, h, e, r0, nb);
}

/* one down tile of 32 * MB rows starting at row r0 (expert e) */
template <int WT, int NS, int MB>
__device__ static void pf_down_tile(uint8_t *lds, int *srow, const _Float16 *h,
				    const uint8_t *down, size_t dn_stride, const int *rows, int E,
				    int EI, float *ypart, int e, int r0, int nb)
{
	constexpr int AL = MB > 2 ? 2 : 1;
	typedef pf_geo<WT, AL> GG;
	constexpr int MT = 32 * MB;
	const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
	const int S = gridDim.z, nst = EI / PF_KB;
	const int s0 = blockIdx.z * nst / S, s1 = (blockIdx.z + 1) * nst / S;
	if (threadIdx.x < MT)
		srow[threadIdx.x] = rows[r0 + threadIdx.x];
	const int n0 = nb * PF_BROWS;
	const size_t RUN = (size_t)PF_BROWS * GG::BB, PANEL = (size_t)E * GG::BB;
	u32 woff[GG::JB];
#pragma unroll
	for (int j = 0; j < GG::JB; j++) {
		const size_t f = (size_t)((wave * GG::JB + j) * WAVE + lane) * GG::CH;
		woff[j] = (u32)((size_t)e * dn_stride +
				(f < 2 * RUN ? (f / RUN) * PANEL + (size_t)n0 * GG::BB + f % RUN
					     : (size_t)n0 * GG::BB));
	}
	pf_lanes2 L;
	u32 aoff[AL];
#pragma unroll
	for (int a = 0; a < AL; a++) {
		const int ar = L.arow + 64 * a;
		aoff[a] = ar < MT && rows[r0 + ar] >= 0
				  ? (u32)((size_t)(r0 + ar) * EI * 2 + 16 * L.achunk)
				  : 0u;
	}
	const int brow[2] = {wave * 64 + 2 * (lane & 31), wave * 64 + 2 * (lane & 31) + 1};
	floatx16 acc[MB < 2 ? 2 : MB][2];
#pragma unroll
	for (int mb = 0; mb < (MB < 2 ? 2 : MB); mb++)
#pragma unroll
		for (int g = 0; g < 2; g++)
#pragma unroll
			for (int j = 0; j < 16; j++)
				acc[mb][g][j] = 0.0f;
	pf_kloop<WT, 1, NS, MB, AL>(lds, down + (size_t)s0 * 2 * PANEL, 2 * PANEL, woff,
				   (const uint8_t *)(h + (size_t)s0 * PF_KB), aoff, brow, s1 - s0,
				   acc); /* syncs srow */
	const int hh = lane >> 5;
#pragma unroll
	for (int mb = 0; mb < MB; mb++)
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const int pr = srow[mb * 32 + 8 * (j / 4) + 4 * hh + (j % 4)];
			if (pr < 0)
				continue;
#pragma unroll
			for (int g = 0; g < 2; g++)
				ypart[((size_t)pr * S + blockIdx.z) * E + n0 + wave * 64 +
				      2 * (lane & 31) + g] = acc[mb][g][j];
		}
}

template <int WT, int NS>
__global__ __launch_bounds__(PF_WAVES * WAVE) void k_pf_down_v(
	const _Float16 *__restrict__ h, const uint8_t *__restrict__ down, size_t dn_stride,
	const int *__restrict__ rows, const int *__restrict__ tinfo, int E, int EI,
	float *__restrict__ ypart)
{
	__shared__ __attribute__((aligned(16))) uint8_t lds[NS * pf_geo<WT, 2>::SSZ];
	__shared__ int srow[128];
	int tile, nb;
	if (!pf_item_v(tinfo[0], tile, nb))
		return;
	const int te = tinfo[1 + 2 * tile], e = te & 0xffff, mb = te >> 16, r0 = tinfo[2 + 2 * tile];
	if (mb == 4)
		pf_down_tile<WT, NS, 4>(lds, srow, h, down, dn_stride, rows, E, EI, ypart, e, r0, nb);
	else if (mb == 2)
		pf_down_tile<WT, NS, 2>(lds, srow, h, down, dn_stride, rows, E, EI, ypart, e, r0, nb);
	else
		pf_down_tile<WT, NS, 1>(lds, srow, h, down, dn_stride, rows, E, EI, ypart, e, r0, nb);
}

/* ---------------------------------------------------------------------- */
/* host                                                                    */
/* ---------------------------------------------------------------------- */

extern "C" int moe_prefill_supported(int wtype, size_t E, size_t EI, size_t NE)
{
	/* offsets from one weights base stay below 4 GB: checked by the caller's
	 * layer size; n-tiles of 256 h columns and 512 output columns */
	return (wtype == 1 || wtype == 2) && NE <= MOE_MAX_NE && E % PF_BROWS == 0 &&
	       EI % (PF_BROWS / 2) == 0 && E % PF_KB == 0 && EI % PF_KB == 0;
}

/* m-tile rows for P pairs over NE experts: 32 while the experts average
 * fewer than 32 pairs */
static int pf_mt(size_t P, size_t NE)
{
	return P < 32 * NE ? 32 : 64;
}

/* tiles a sort of P pairs into MT-row tiles can use */
static size_t pf_tiles(size_t P, size_t NE, size_t mt)
{
	return (P + mt - 1) / mt + (NE < P ? NE : P);
}

/* tiles and rows of k_moe_sort_v for P pairs: an expert of c pairs takes at
 * most c / 128 + 1 tiles and c + 63 rows */
static size_t pf_vtiles(size_t P, size_t NE)
{
	return P / 128 + (NE < P ? NE : P) + 1;
}

static size_t pf_vrows(size_t P, size_t NE)
{
	return P + 64 * (NE < P ? NE : P);
}

/* capacities for every call of at most P pairs (32-row tiles below 32 pairs
 * per expert, variable tiles from there; each term grows with P, so a
 * smaller call always fits) */
extern "C" int moe_prefill_max_tiles(size_t P, size_t NE)
{
	const size_t p32 = P < 32 * NE ? P : 32 * NE;
	const size_t a = pf_vtiles(P, NE), b = pf_tiles(p32, NE, 32);
	return (int)(a > b ? a : b);
}

extern "C" size_t moe_prefill_max_rows(size_t P, size_t NE)
{
	const size_t p32 = P < 32 * NE ? P : 32 * NE;
	const size_t a = pf_vrows(P, NE), b = pf_tiles(p32, NE, 32) * 32;
	return a > b ? a : b;
}

/* ints of the tile table: 32-row tiles keep one per tile plus the count,
 * variable tiles two per tile plus the count */
extern "C" size_t moe_prefill_tile_ints(size_t P, size_t NE)
{
	return 2 * (size_t)moe_prefill_max_tiles(P, NE) + 1;
}

/* the largest tile table the sort kernel handles */
extern "C" int moe_prefill_tile_cap(void)
{
	return SORT_MAX_TILES;
}

extern "C" int moe_launch_prefill(int wtype, const void *xh_, const uint8_t *gate,
				  const uint8_t *up, const uint8_t *down, size_t gu_stride,
				  size_t dn_stride, const uint32_t *ids, int *rows, int *tile_e,
				  void *h16, float *ypart, int T, int K, int E, int EI, int NE,
				  int max_split, int *split, void *stream)
{
	if (!moe_prefill_supported(wtype, (size_t)E, (size_t)EI, (size_t)NE) || up < gate)
		return (int)hipErrorInvalidValue;
	const size_t up_off = (size_t)(up - gate);
	/* every weight offset a lane forms must fit 32 bits */
	if (up_off + (size_t)NE * gu_stride > 0xffffffffull ||
	    (size_t)NE * dn_stride > 0xffffffffull ||
	    (size_t)T * E * 2 > 0xffffffffull)
		return (int)hipErrorInvalidValue;
	hipStream_t s = (hipStream_t)stream;
	const _Float16 *xh = (const _Float16 *)xh_;
	const int P = T * K;
	const int mt = pf_mt((size_t)P, (size_t)NE);
	if (mt == 64) { /* many pairs per expert: tiles of 32, 64 or 128 rows */
		const int Tv = (int)pf_vtiles((size_t)P, (size_t)NE);
		if (Tv > 65535 || pf_vrows((size_t)P, (size_t)NE) * EI * 2 > 0xffffffffull)
			return (int)hipErrorInvalidValue;
		hipLaunchKernelGGL(k_moe_sort_v, dim3(1), dim3(SORT_THREADS), 0, s, ids, P, NE, Tv,
				   rows, tile_e);
		_Float16 *hh = (_Float16 *)h16;
		const int nx = E / PF_BROWS, nst = EI / PF_KB;
		int S = 512 / (nx * Tv);
		if (S > max_split)
			S = max_split;
		if (S > nst / 8)
			S = nst / 8;
		if (S < 1)
			S = 1;
		*split = S;
		const dim3 ggu(EI / (PF_BROWS / 2), Tv), gdn(nx, Tv, S), blk(PF_WAVES * WAVE);
		/* one workgroup per CU: gate/up Q4_0 4 stages of 40 KB (3 in flight:
		 * 79.4 -> 76.6 us against 3 stages at OLMoE T=512), down 3 (its
		 * row table takes LDS too); Q8_0 2 of 56 KB */
		if (wtype == 1) {
			hipLaunchKernelGGL((k_pf_gateup_v<1, 2>), ggu, blk, 0, s, xh, gate, up_off,
					   gu_stride, rows, tile_e, K, E, EI, hh);
			hipLaunchKernelGGL((k_pf_down_v<1, 2>), gdn, blk, 0, s, hh, down, dn_stride, rows,
					   tile_e, E, EI, ypart);
		} else {
			hipLaunchKernelGGL((k_pf_gateup_v<2, 4>), ggu, blk, 0, s, xh, gate, up_off,
					   gu_stride, rows, tile_e, K, E, EI, hh);
			hipLaunchKernelGGL((k_pf_down_v<2, 3>), gdn, blk, 0, s, hh, down, dn_stride, rows,
					   tile_e, E, EI, ypart);
		}
		return (int)hipGetLastError();
	}
	const int Tmax = (int)pf_tiles((size_t)P, (size_t)NE, (size_t)mt);
	if (Tmax > SORT_MAX_TILES || (size_t)Tmax * mt * EI * 2 > 0xffffffffull)
		return (int)hipErrorInvalidValue;
	if (mt == 32)
		hipLaunchKernelGGL(k_moe_sort<32>, dim3(1), dim3(SORT_THREADS), 0, s, ids, P, NE, Tmax,
				   rows, tile_e);
	else
		hipLaunchKernelGGL(k_moe_sort<64>, dim3(1), dim3(SORT_THREADS), 0, s, ids, P, NE, Tmax,
				   rows, tile_e);
	_Float16 *hh = (_Float16 *)h16;
	/* split the down projection's K when its (m-tile, column block) grid
	 * would leave most CUs idle (few tokens per expert, large d_ff), aiming
	 * at two workgroups per CU.  Tiles counted: with 32-row tiles nearly
	 * every touched expert has one, so the experts touched (Mixtral T=64:
	 * 8, where the bound says 12; 207.9 -> 200.6 us); with 64-row tiles
	 * the bound, since skewed experts add ragged tails (counting fewer
	 * measured 8% slower at OLMoE T=512). */
	const int nx = E / PF_BROWS, nst = EI / PF_KB;
	const int tiles = mt == 32 ? max((P + mt - 1) / mt, min(NE, P)) : Tmax;
	int S = 512 / (nx * tiles);
	if (S > max_split)
		S = max_split;
	if (S > nst / 8)
		S = nst / 8;
	if (S < 1)
		S = 1;
	*split = S;
	const dim3 ggu(EI / (PF_BROWS / 2), Tmax), gdn(nx, Tmax, S);
	const dim3 blk(PF_WAVES * WAVE);
#define PF_LAUNCH(W, NS, MB)                                                                 \
	do {                                                                                 \
		hipLaunchKernelGGL((k_pf_gateup<W, NS, MB>), ggu, blk, 0, s, xh, gate, up_off,    \
				   gu_stride, rows, tile_e, K, E, EI, hh);                        \
		hipLaunchKernelGGL((k_pf_down<W, NS, MB>), gdn, blk, 0, s, hh, down, dn_stride,   \
				   rows, tile_e, E, EI, ypart);                                   \
	} while (0)
	if (wtype == 1) { /* 3 stages (144 KB): one workgroup per CU */
		if (mt == 32)
			PF_LAUNCH(1, 3, 1);
		else
			PF_LAUNCH(1, 3, 2);
	} else {
		/* two 2-stage workgroups per CU, one dequantizing while the other
		 * runs its MFMAs; it also fits grids of 1.5-2 workgroups per CU
		 * (Mixtral T=16/64) in one round.  Measured against one 4-stage
		 * workgroup per CU for tiles of mostly padding rows: Mixtral T=64
		 * 342.4 -> 337.4 us, T=16 330.3 -> 326.8 us. */
		if (mt == 32)
			PF_LAUNCH(2, 2, 1);
		else
			PF_LAUNCH(2, 2, 2);
	}
#undef PF_LAUNCH
	return (int)hipGetLastError();
}
