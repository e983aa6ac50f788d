/*
 * Device helpers shared by the MoE kernels (gfx950, wave64).
 *
 * Weights stay in GGUF block layout (Q8_0: 34-byte blocks, Q4_0: 18-byte
 * blocks, quant.h:14-26).  A lane owns a "segment" of two consecutive blocks
 * (64 columns: 68 bytes Q8_0 / 36 bytes Q4_0, always 4-byte aligned because
 * rows hold an even number of blocks) and keeps the matching 64 activations in
 * registers for all the rows it visits; C lanes cover one row (or one K-chunk
 * of a row), 64/C rows are in flight per wave step, and a row's partial sums
 * meet in an xor-shuffle tree.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add is written.
 */
#ifndef MOE_DEVICE_H
#define MOE_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_expf.h"
#include "moe_internal.h"

typedef uint32_t u32;

#define WAVE 64

/* LDS ordering between lanes of one wave (no workgroup barrier). */
#define WAVE_SYNC()                                              \
	do {                                                     \
		__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront"); \
		__builtin_amdgcn_wave_barrier();                 \
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront"); \
	} while (0)

__device__ static inline float f16_bits_to_f32(u32 h)
{
	return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

/* One LDS-DMA load per lane (global_load_lds_dwordx4): 16 bytes from
 * sbase + voff into LDS at lds + 16 * lane (lds wave-uniform).  Issued from
 * inline assembly, so the compiler's own waits do not count it (its
 * conservative wait for every LDS-DMA write before any LDS read would undo
 * the kernels' multi-stage buffering): callers wait with wait_vm.  The LDS
 * address goes in as an m0 operand, so the compiler writes m0 itself and
 * knows it does; the s_nop is the one wait state an m0 write needs before
 * an LDS-DMA instruction. */
__device__ static inline void dma_dwordx4(const void *sbase, u32 voff, u32 lds)
{
	/* the base is wave-uniform by contract: pinned to SGPRs (the builtin
	 * returns int: each half goes through u32, so none is sign-extended) */
	const uint64_t b = (uint64_t)(uintptr_t)sbase;
	const uint64_t bs = (uint64_t)(u32)__builtin_amdgcn_readfirstlane((int)(u32)b) |
			    ((uint64_t)(u32)__builtin_amdgcn_readfirstlane((int)(u32)(b >> 32)) << 32);
	asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
		     :
		     : "v"(voff), "s"((const void *)(uintptr_t)bs),
		       "{m0}"(__builtin_amdgcn_readfirstlane(lds))
		     : "memory");
}

/* wait until at most N of this wave's vector memory operations are pending
 * (loads return in order, so the older ones are then complete) */
template <int N>
__device__ static inline void wait_vm()
{
	static_assert(N >= 0 && N < 64, "vmcnt is six bits");
	__builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

/* the LDS address of a shared-memory pointer */
__device__ static inline u32 lds_addr(const void *p)
{
	return (u32)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
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

/*
 * Dequant dots.  A quant byte is converted with v_cvt_f32_ubyte*: for Q8_0
 * the byte b is read as (b ^ 0x80) = q + 128, for Q4_0 a nibble n = q + 8, so
 *   sum_i q_i x_i = sum_i (q_i + c) x_i - c * sum_i x_i
 * with the block's sum_i x_i (xs) computed once per lane and reused for
 * every row.  Two VALU operations per weight instead of four or five.
 */

/* the sum of 32 consecutive floats */
__device__ static inline float sum32(const float *x)
{
	float s = 0.0f;
#pragma unroll
	for (int i = 0; i < 32; i++)
		s += x[i];
	return s;
}

/* acc + sum over the 4 bytes of u of byte_j * x[j] */
__device__ static inline float fma_ubytes(u32 u, const float *x, float acc)
{
	acc = __builtin_fmaf((float)(u & 0xffu), x[0], acc);
	acc = __builtin_fmaf((float)((u >> 8) & 0xffu), x[1], acc);
	acc = __builtin_fmaf((float)((u >> 16) & 0xffu), x[2], acc);
	acc = __builtin_fmaf((float)(u >> 24), x[3], acc);
	return acc;
}

/* Q8_0 block: 8 dwords of quants q0..q31 (already aligned), scale bits */
__device__ static inline float block_dot_q8_0(const u32 (&q)[8], u32 dbits, const float *x,
					      float xs)
{
	float acc = 0.0f;
#pragma unroll
	for (int k = 0; k < 8; k++)
		acc = fma_ubytes(q[k] ^ 0x80808080u, x + 4 * k, acc);
	return f16_bits_to_f32(dbits) * __builtin_fmaf(-128.0f, xs, acc);
}

/* Q4_0 block: 4 dwords of packed bytes (element j low nibble of byte j,
 * element j+16 high nibble), scale bits */
__device__ static inline float block_dot_q4_0(const u32 (&q)[4], u32 dbits, const float *x,
					      float xs)
{
	float acc = 0.0f;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		acc = fma_ubytes(q[k] & 0x0f0f0f0fu, x + 4 * k, acc);
		acc = fma_ubytes((q[k] >> 4) & 0x0f0f0f0fu, x + 16 + 4 * k, acc);
	}
	return f16_bits_to_f32(dbits) * __builtin_fmaf(-8.0f, xs, acc);
}

/* Q8_0 segment: 17 dwords.  Block 0 = bytes 0..33 (scale in bytes 0-1,
 * quants 2..33, i.e. misaligned by 2), block 1 = bytes 34..67 (scale 34-35,
 * quants 36..67 = dwords 9..16).  xs0, xs1: sums of x[0..31], x[32..63]. */
__device__ static inline float seg_dot_q8_0(const u32 (&d)[17], const float (&x)[64], float xs0,
					    float xs1)
{
	u32 q0[8], q1[8];
#pragma unroll
	for (int k = 0; k < 8; k++) {
		q0[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		q1[k] = d[9 + k];
	}
	return block_dot_q8_0(q0, d[0], x, xs0) + block_dot_q8_0(q1, d[8] >> 16, x + 32, xs1);
}

/* Q4_0 segment: 9 dwords.  Block 0 = bytes 0..17 (scale 0-1, packed nibbles
 * 2..17), block 1 = bytes 18..35 (scale 18-19, nibbles 20..35 = dwords 5..8).
 * Byte j of a block holds element j (low nibble) and j+16 (high nibble),
 * each biased by 8 (quant.c:126-155). */
__device__ static inline float seg_dot_q4_0(const u32 (&d)[9], const float (&x)[64], float xs0,
					    float xs1)
{
	u32 q0[4], q1[4];
#pragma unroll
	for (int k = 0; k < 4; k++) {
		q0[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		q1[k] = d[5 + k];
	}
	return block_dot_q4_0(q0, d[0], x, xs0) + block_dot_q4_0(q1, d[4] >> 16, x + 32, xs1);
}

/*
 * One block of a down-matrix panel.  The layer keeps each down matrix as
 * EI/32 panels: panel c holds block c of every row, row i's at BB*i.  The
 * 4-byte aligned window that holds it starts 2 bytes early for odd i (scale
 * in the upper half of dword 0) and runs 2 bytes into block i+1 for even i;
 * E is even, so the last row is odd and no window leaves its panel.
 */
template <int WT> struct panel_blk;
template <> struct panel_blk<1> { /* Q8_0 */
	static constexpr int BB = 34, DW = 9;
	__device__ static inline float dot(const u32 (&d)[9], int i, const float *h, float hs)
	{
		u32 q[8];
		const bool odd = i & 1;
#pragma unroll
		for (int k = 0; k < 8; k++)
			q[k] = odd ? d[k + 1] : __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		return block_dot_q8_0(q, odd ? d[0] >> 16 : d[0], h, hs);
	}
};
template <> struct panel_blk<2> { /* Q4_0 */
	static constexpr int BB = 18, DW = 5;
	__device__ static inline float dot(const u32 (&d)[5], int i, const float *h, float hs)
	{
		u32 q[4];
		const bool odd = i & 1;
#pragma unroll
		for (int k = 0; k < 4; k++)
			q[k] = odd ? d[k + 1] : __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		return block_dot_q4_0(q, odd ? d[0] >> 16 : d[0], h, hs);
	}
};

template <int WT> struct qseg;
template <> struct qseg<1> {
	static constexpr int BYTES = 68;
	static constexpr int DW = 17;
	__device__ static inline float dot(const uint8_t *p, const float (&x)[64], float xs0,
					   float xs1)
	{
		u32 d[17];
		load_dwords<17>(p, d);
		return seg_dot_q8_0(d, x, xs0, xs1);
	}
};
template <> struct qseg<2> {
	static constexpr int BYTES = 36;
	static constexpr int DW = 9;
	__device__ static inline float dot(const uint8_t *p, const float (&x)[64], float xs0,
					   float xs1)
	{
		u32 d[9];
		load_dwords<9>(p, d);
		return seg_dot_q4_0(d, x, xs0, xs1);
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

/* device-coherent accesses (global_{load,store} ... sc1) */
__device__ static inline void st_dev_u32(u32 *p, u32 v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline void st_dev_u64(uint64_t *p, uint64_t v)
{
	__hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

/* Activations staged in LDS with 4 floats of padding after every 64-float
 * segment, so the C lanes of a row group reading their segments with 16-byte
 * LDS reads hit distinct banks. */
#define SEG_STRIDE 68

__device__ static inline void lds_x64(const float *s, int seg, float (&x)[64])
{
	const float4 *s4 = (const float4 *)(s + seg * SEG_STRIDE);
#pragma unroll
	for (int i = 0; i < 16; i++) {
		float4 v = s4[i];
		x[4 * i + 0] = v.x;
		x[4 * i + 1] = v.y;
		x[4 * i + 2] = v.z;
		x[4 * i + 3] = v.w;
	}
}

/* Copy n floats (n a multiple of 64) from global into the padded LDS
 * layout, all threads of a block of nthreads cooperating. */
__device__ static inline void stage_padded(float *s, const float *g, int n, int tid,
					   int nthreads)
{
	const float4 *g4 = (const float4 *)g;
	for (int i = tid; i < n / 4; i += nthreads) {
		float4 v = g4[i];
		*(float4 *)(s + (i >> 4) * SEG_STRIDE + (i & 15) * 4) = v;
	}
}

/*
 * softmax_1d + top_k (+ Mixtral renormalisation) for one token, one wave.
 *
 * softmax_1d (nn.c:221-262): e_i = expf(v_i - max); lane sums s_l over the
 * 8-wide chunks in order, the reduction tree ((s0+s4)+(s2+s6))+((s1+s5)+
 * (s3+s7)), then the scalar tail; p_i = e_i / sum (IEEE division).
 *
 * top_k (nn.c:276-308) seeds all k slots with element 0 and inserts later
 * elements only when strictly greater than the current minimum.  Its result
 * in closed form: rank_i = #{j : p_j > p_i or (p_j == p_i and j < i)};
 * r0 = rank of element 0.  Element i != 0 lands in slot k-1-rank_i iff
 * rank_i < min(r0, k); when r0 < k, slots 0..k-1-r0 hold copies of element 0.
 * Slots ascend by weight, later indices below earlier ones among ties.
 *
 * renorm (llama.c:422-427): w_e /= (sequential sum of the k weights).
 * sp holds NE floats and sid/sw K entries of this wave's LDS.
 */
__device__ static inline void wave_softmax_topk(const float *logits, float *probs, u32 *ids,
						float *wout, int NE, int K, int renorm,
						float *sp, u32 *sid, float *sw, int lane)
{
	float mx = -__builtin_inff();
	for (int i = lane; i < NE; i += WAVE)
		mx = fmaxf(mx, logits[i]);
#pragma unroll
	for (int off = 32; off >= 1; off >>= 1)
		mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));

	for (int i = lane; i < NE; i += WAVE)
		sp[i] = moe_expf(logits[i] - mx);
	WAVE_SYNC();

	const int nv = NE - NE % 8;
	float ev[MOE_MAX_NE / WAVE];
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++)
		ev[r] = (lane + r * WAVE < NE) ? sp[lane + r * WAVE] : 0.0f;
	/* lane l < 8: s_l = e_l + e_{8+l} + e_{16+l} + ... in order; element
	 * 8c+l sits in ev[c/8] of lane 8(c%8)+l */
	float s = 0.0f;
#pragma unroll
	for (int c = 0; c < MOE_MAX_NE / 8; c++) {
		float v = __shfl(ev[c >> 3], 8 * (c & 7) + (lane & 7), WAVE);
		if (8 * c < nv)
			s = s + v;
	}
	s = s + __shfl_xor(s, 4, 8);
	s = s + __shfl_xor(s, 2, 8);
	s = s + __shfl_xor(s, 1, 8);
	for (int i = nv; i < NE; i++)
		s += sp[i];
	const float sum = __shfl(s, 0, WAVE);

	float pv[MOE_MAX_NE / WAVE];
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
		int i = lane + r * WAVE;
		pv[r] = 0.0f;
		if (i < NE) {
			pv[r] = ev[r] / sum;
			if (probs)
				probs[i] = pv[r];
		}
	}

	/* rank_i over broadcasts of every p_j (v_readlane, no memory round trip) */
	int rank[MOE_MAX_NE / WAVE];
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++)
		rank[r] = 0;
#pragma unroll
	for (int r2 = 0; r2 < MOE_MAX_NE / WAVE; r2++) {
		if (r2 * WAVE >= NE)
			break;
		const int pbits = __builtin_bit_cast(int, pv[r2]);
		const int n2 = NE - r2 * WAVE < WAVE ? NE - r2 * WAVE : WAVE;
		for (int j2 = 0; j2 < n2; j2++) {
			const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(pbits, j2));
			const int j = r2 * WAVE + j2;
#pragma unroll
			for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
				const int i = lane + r * WAVE;
				rank[r] += (pj > pv[r]) || (pj == pv[r] && j < i);
			}
		}
	}
	WAVE_SYNC();
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
		int i = lane + r * WAVE;
		if (i < NE)
			sp[i] = pv[r];
	}
	WAVE_SYNC();
	const int r0 = __shfl(rank[0], 0, WAVE);
	const int lim = r0 < K ? r0 : K;
#pragma unroll
	for (int r = 0; r < MOE_MAX_NE / WAVE; r++) {
		int i = lane + r * WAVE;
		if (i > 0 && i < NE && rank[r] < lim) {
			sid[K - 1 - rank[r]] = (u32)i;
			sw[K - 1 - rank[r]] = pv[r];
		}
	}
	if (r0 < K) {
		float p0 = sp[0];
		for (int slot = lane; slot < K - r0; slot += WAVE) {
			sid[slot] = 0;
			sw[slot] = p0;
		}
	}
	WAVE_SYNC();
	if (lane == 0 && renorm) {
		float ws = 0.0f;
		for (int e = 0; e < K; e++)
			ws += sw[e];
		for (int e = 0; e < K; e++)
			sw[e] /= ws;
	}
	WAVE_SYNC();
	for (int e = lane; e < K; e += WAVE) {
		ids[e] = sid[e];
		wout[e] = sw[e];
	}
}

/* DPP lane moves (VALU, no LDS round trip).  Controls: quad_perm [1,0,3,2]
 * = 0xb1, [2,3,0,1] = 0x4e, row_shl:n = 0x100 + n, row_mirror = 0x140,
 * row_half_mirror = 0x141.  Lanes whose source falls outside their row of 16
 * read 0. */
template <int CTRL>
__device__ static inline float dpp_f32(float v)
{
	return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
								     CTRL, 0xf, 0xf, false));
}

__device__ static inline float lane_f32(float v, int l)
{
	return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

/* max over the wave, in every lane (max is exact, so any order) */
__device__ static inline float wave_max_f32(float v)
{
	v = fmaxf(v, dpp_f32<0xb1>(v));  /* lane ^ 1 */
	v = fmaxf(v, dpp_f32<0x4e>(v));  /* lane ^ 2 */
	v = fmaxf(v, dpp_f32<0x141>(v)); /* the other quad of the 8 */
	v = fmaxf(v, dpp_f32<0x140>(v)); /* the other 8 of the row */
	return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

/*
 * wave_softmax_topk for NE <= 64: element i lives in lane i.  Same arithmetic
 * and order as wave_softmax_topk: max, e = expf(x - max), lane sums
 * s_l = e_l + e_{l+8} + ... in order, the tree ((s0+s4)+(s2+s6)) +
 * ((s1+s5)+(s3+s7)) (vector_avx2.h:126-132), the scalar tail, p = e / sum.
 * softmax64 returns p and the lane's rank key; keys order like the
 * probabilities, ties broken towards the lower index:
 * key = (bits(p) + 1) << 6 | (63 - index), 0 for lanes past NE.
 */
__device__ static inline float softmax64(float logit, int NE, const uint64_t *tab, int lane,
					 uint64_t &key)
{
	const bool valid = lane < NE;
	const float mx = wave_max_f32(valid ? logit : -__builtin_inff());
	const float e = valid ? moe_expf_tab(logit - mx, tab) : 0.0f;

	const int nv = NE - NE % 8;
	float g[8];
#pragma unroll
	for (int c = 0; c < 8; c++)
		g[c] = __shfl(e, 8 * c + (lane & 7), WAVE);
	float s = 0.0f;
#pragma unroll
	for (int c = 0; c < 8; c++)
		if (8 * c < nv)
			s = s + g[c];
	s = s + dpp_f32<0x104>(s); /* lane l: s_l + s_{l+4} */
	s = s + dpp_f32<0x102>(s); /* + the pair two lanes up */
	s = s + dpp_f32<0x101>(s); /* lane 0: the full tree */
	float sum = lane_f32(s, 0);
	for (int i = nv; i < NE; i++)
		sum += lane_f32(e, i);
	const float p = e / sum;
	/* p >= 0, so its bits order like the values: j beats i iff key_j > key_i */
	key = valid ? ((uint64_t)(__builtin_bit_cast(u32, p) + 1u) << 6) | (uint64_t)(63 - lane) : 0;
	return p;
}

/* number of the n keys sk[0..n) (LDS, read as broadcasts) above key */
__device__ static inline int rank_part64(const uint64_t *sk, int n, uint64_t key)
{
	int rank = 0;
	const ulonglong2 *sk2 = (const ulonglong2 *)sk;
	for (int q = 0; q < n / 2; q++) {
		const ulonglong2 v = sk2[q];
		rank += (int)(v.x > key);
		rank += (int)(v.y > key);
	}
	return rank;
}

/*
 * top_k (nn.c:276-308) from the ranks: element i != 0 lands in slot k-1-rank_i
 * iff rank_i < min(rank_0, k); the slots left over hold element 0 (every slot
 * is seeded with it and only strictly greater values are inserted).  Then
 * the Mixtral renorm (sequential sum, then divide: llama.c:422-427).  sid/sw
 * are k entries of this wave's LDS; ids/w receive the slots (LDS or global).
 */
__device__ static inline void topk_finish64(int rank, float p, u32 *ids, float *wout, int NE,
					    int K, int renorm, u32 *sid, float *sw, int lane)
{
	const bool valid = lane < NE;
	const int r0 = __builtin_amdgcn_readlane(rank, 0);
	const int lim = r0 < K ? r0 : K;
	if (lane > 0 && valid && rank < lim) {
		sid[K - 1 - rank] = (u32)lane;
		sw[K - 1 - rank] = p;
	}
	const float p0 = lane_f32(p, 0);
	if (r0 < K)
		for (int slot = lane; slot < K - r0; slot += WAVE) {
			sid[slot] = 0;
			sw[slot] = p0;
		}
	WAVE_SYNC();
	if (lane == 0 && renorm) {
		float ws = 0.0f;
		for (int k = 0; k < K; k++)
			ws += sw[k];
		for (int k = 0; k < K; k++)
			sw[k] /= ws;
	}
	WAVE_SYNC();
	for (int k = lane; k < K; k += WAVE) {
		ids[k] = sid[k];
		wout[k] = sw[k];
	}
}

/* all of it in one wave: sp 128 floats of this wave's LDS (8-byte aligned) */
__device__ static inline void wave_softmax_topk64(float logit, u32 *ids, float *wout, int NE,
						  int K, int renorm, const uint64_t *tab,
						  float *sp, u32 *sid, float *sw, int lane)
{
	uint64_t key;
	const float p = softmax64(logit, NE, tab, lane, key);
	uint64_t *sk = (uint64_t *)sp;
	sk[lane] = key;
	WAVE_SYNC();
	const int rank = rank_part64(sk, 64, key);
	topk_finish64(rank, p, ids, wout, NE, K, renorm, sid, sw, lane);
}

#endif
