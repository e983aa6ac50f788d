/*
 * Decode-sized MoE FFN layer (up to MOE_FUSED_MAX_P token-slot pairs) in one
 * launch: k_moe_decode.
 *
 * One workgroup per CU, all G of them resident.  The unit of work ("item")
 * is one (token, slot) pair p and one chunk c of DEC_CHUNK = 32 rows of
 * d_ff.  An item streams
 *   - rows 32c .. 32c+31 of the gate and up matrices of expert e = ids[p]
 *     (GGUF rows, contiguous in memory), and
 *   - panel c of the expert's down matrix: block c of each of its E rows
 *     (the layer keeps down matrices panel by panel, so these E blocks are
 *     contiguous too),
 * computes h = silu(gate.x) * (up.x) for its 32 rows (nn.c:460-478) into
 * LDS, then the contribution of those 32 columns of down to all E outputs,
 * scaled the way the combine scales a slot, y / (1/w) (olmoe.c:401-403).
 * No item waits for another one, so a workgroup streams the weights of its
 * items back to back, the next item's loads in flight while the current
 * one computes.
 *
 * Phases of workgroup b:
 *  1. routing.  Workgroup j < NE computes router logit j for every token
 *     with the 8-lane FMA chains of dot_f32_f32 (matmul.c:91-105), fed from
 *     LDS-transposed copies of router row j and the token, and writes it into
 *     NREP replicas of the logit table, each entry tagged with this launch's
 *     epoch.  Every workgroup polls its own replica (lane j of a wave polls
 *     expert j of a token; the loads that see the epoch deliver the logits)
 *     and runs softmax + top-k (+ renorm) itself (nn.c:221-308,
 *     llama.c:422-427).  The tokens its items need are staged into LDS
 *     meanwhile.
 *  2. items: a balanced contiguous range of the T*K*(EI/32) items in
 *     (token, slot, chunk) order, dealt in half items (16 rows of d_ff) so
 *     that shares stay equal when the items do not divide evenly over the
 *     workgroups; a half streams its 16 gate/up rows and the whole down
 *     panel.  One workgroup's items belong to at most DEC_TOKS tokens.
 *     Thread i accumulates outputs i, i + NT, ... of a token over its items
 *     in registers and publishes them once per token as epoch-tagged
 *     partials.
 *  3. combine.  The T*E outputs form slices of PSLICE; for each of its slices
 *     a workgroup polls the partials of every workgroup holding items of the
 *     slice's token (one hop: the loads that see the epoch deliver the
 *     values) and adds them in a fixed order.
 *  4. epoch.  Each workgroup raises a start flag once it has read the epoch
 *     word; workgroup 0, when done, checks them and advances the epoch for
 *     the next launch (which starts after this one drains).
 *
 * Synchronisation uses no read-modify-write: producers write epoch-tagged
 * words and consumers poll them.  The only waits are the routing (on the NE
 * router workgroups) and the combine (on every workgroup with items), so
 * the grid must be resident: one workgroup per CU.  Waits are bounded
 * regardless; one that runs out sets an error word instead of hanging.
 *
 * Data produced by another workgroup in the same launch (logits, partials)
 * is written with device-coherent stores (agent-scope relaxed atomics: `sc1`
 * on gfx950, written through the per-XCD L2) and read with device-coherent
 * loads.  Agent-scope release/acquire fences are avoided: on gfx950 they
 * write back / invalidate a whole XCD L2.
 *
 * Weights stay in GGUF blocks.  Gate/up: a lane owns one segment of a row,
 * Q8_0 one 34-byte block (9 dwords loaded from the 4-byte aligned window
 * that holds it, 32 columns), Q4_0 a pair of 18-byte blocks (9 dwords, 64
 * columns), and the matching activations.  Down: a lane owns whole rows of
 * the panel, one block each, and the item's 32 h values.
 */
#include "moe_device.h"
#include "kq_device.h"

#include <pthread.h>

#define NREP 64      /* == WAVE: one replica per lane of the writing wave */
#define PSLICE 8     /* outputs per combine slice */
#define DEC_TOKS 2   /* tokens one workgroup's item range can span (T <= G) */
#define DEC_CHUNK 32 /* d_ff rows per item: one down block per row */
#define CMB_MAX 16   /* combine entries per thread, two slices: grid * PSLICE <= CMB_MAX / 2 * NT */

/* Stage stamps (a build with -DMOE_STAGE_STAMPS only, libhip_moe_stamps.so):
 * thread 0 of each workgroup writes the 100 MHz wall clock at its start,
 * after routing, after its last item's gate/up, after its partials, and
 * after the combine, into a device array that moe_stage_stamps copies out.
 * The product library compiles the stamps to nothing. */
#define MOE_STAMP_WGS 1024
#define MOE_STAMPS 5
#ifdef MOE_STAGE_STAMPS
__device__ unsigned long long g_stage_stamps[MOE_STAMP_WGS * MOE_STAMPS];
#define STAMP(k)                                                                           \
	do {                                                                               \
		if (threadIdx.x == 0 && blockIdx.x < MOE_STAMP_WGS)                         \
			g_stage_stamps[blockIdx.x * MOE_STAMPS + (k)] = wall_clock64();      \
	} while (0)
#else
#define STAMP(k) \
	do {     \
	} while (0)
#endif

struct DecodeArgs {
	const float *x;
	const float *router;
	const float *bias;
	const uint8_t *gate, *up, *down;
	size_t gu_stride, dn_stride;
	u32 *ids_out;
	float *w_out;
	uint64_t *part; /* [T][E / PSLICE][ncon][PSLICE], epoch-tagged */
	float *out;
	u32 *sync;
	int T, E, EI, NE, K, renorm;
	int n_items, ncon;
	int off_start, off_rep;
	int rep_stride; /* u64 entries between replicas (a multiple of 512: 4 KB) */
	int spin;       /* poll rounds after which a wait gives up (MOE_SPIN_DEFAULT) */
	/* k_moe_decode<..., NORM = true> (one token): x is the residual h, the
	 * layer's input rms_norm(h) * norm_w, which router workgroup 0 also
	 * writes to x_out */
	const float *norm_w;
	float *x_out;
};

/* balanced split of n items over G workgroups: b gets [item_lo(b), item_lo(b+1));
 * n * G < 2^31 (n <= 64 pairs * 2048 chunks, G <= 4096) */
__host__ __device__ static inline int item_lo(int b, int n, int G)
{
	return (int)((unsigned)b * (unsigned)n / (unsigned)G);
}

/* the workgroup whose range holds item x (0 <= x < n): the largest b with
 * item_lo(b) <= x, which is never an empty range */
__host__ __device__ static inline int item_owner(int x, int n, int G)
{
	return (int)(((unsigned)(x + 1) * (unsigned)G + (unsigned)n - 1) / (unsigned)n) - 1;
}

/*
 * The whole workgroup waits until n flags starting at f all equal `epoch`.
 * Each thread checks n / NT of them per round.
 */
template <int NT>
__device__ static inline bool wait_flags(const u32 *f, int n, u32 epoch, u32 *err, u32 code,
					 int spin)
{
	__shared__ int s_ok;
	int step = 0;
	for (int round = 0;; round++) {
		bool ok = true;
		for (int i = threadIdx.x; i < n; i += NT)
			ok &= ld_dev_u32(&f[i]) == epoch;
		if (threadIdx.x == 0)
			s_ok = 1;
		__syncthreads();
		if (!ok)
			s_ok = 0;
		__syncthreads();
		if (s_ok)
			return true;
		if (round >= spin) {
			if (threadIdx.x == 0)
				st_dev_u32(err, code);
			return false;
		}
		backoff(step);
		__syncthreads();
	}
}

/* ---------------------------------------------------------------------- */
/* blocks                                                                 */
/* ---------------------------------------------------------------------- */

template <int WT> struct segq;

/* gate/up, Q8_0: one block per lane.  Block s of a row starts at byte 34s;
 * the 36-byte window starting at (34s & ~3) holds it: scale in bytes 0-1 of
 * the window (even s) or 2-3 (odd s), quants right after. */
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

/* gate/up, Q4_0: a pair of blocks per lane, 36 bytes at 36s (quant.c:126-155). */
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

/* ---------------------------------------------------------------------- */
/* integer dots                                                           */
/* ---------------------------------------------------------------------- */

/*
 * An activation block (32 values of a token, or an item's 32 h values) is
 * held as X_k = rint(v_k * 2^s), s chosen per block so |X_k| < 2^22, split
 * into three balanced signed base-256 digits X = D2*65536 + D1*256 + D0
 * (each in [-128, 127]).  A weight block's quants meet the digits in
 * v_dot4c_i32_i8 (four products per instruction, exact int32 sums), and
 *   sum q*v = 2^-s * (65536*S2 + (256*S1 + S0)),
 * rounded once when the two parts meet in fp32.  The rounding of v to 22
 * bits below its block's largest magnitude keeps a dot within ~1e-6 of the
 * fp32 one; the reference's own fp32 sums differ by as much.  One weight
 * byte costs 3/4 of an instruction instead of a conversion and an FMA.
 *
 * A staged block is DBLK dwords: d2[8] d1[8] d0[8] (element 4k+i in byte i
 * of dword k), 2^-s, and the block sums of each digit (Q4_0 stores q + 8).
 */
#define DBLK 28

__device__ static inline int digit_lo(int &x)
{
	const int d = ((x + 128) & 255) - 128;
	x = (x - d) >> 8;
	return d;
}

/* 4 values of a block held by one of its 8 staging lanes (lanes 8j..8j+7 of
 * a wave hold block j): the block's digits and scale into dst[DBLK] */
__device__ static inline void stage_digits4(u32 *dst, float4 v, int sub)
{
	float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
	m = fmaxf(m, __shfl_xor(m, 1, 8));
	m = fmaxf(m, __shfl_xor(m, 2, 8));
	m = fmaxf(m, __shfl_xor(m, 4, 8));
	/* 2^s * m < 2^22; a block of zeros (or denormals) takes s = 120 */
	const int e = (int)((__builtin_bit_cast(u32, m) >> 23) & 0xffu) - 127;
	const int sh = 21 - e < 120 ? 21 - e : 120;
	const float sc = __builtin_bit_cast(float, (u32)(sh + 127) << 23);
	const float vv[4] = {v.x, v.y, v.z, v.w};
	u32 p2 = 0, p1 = 0, p0 = 0;
	int s2 = 0, s1 = 0, s0 = 0;
#pragma unroll
	for (int i = 0; i < 4; i++) {
		int x = __float2int_rn(vv[i] * sc);
		const int d0 = digit_lo(x), d1 = digit_lo(x), d2 = x;
		p0 |= (u32)(d0 & 255) << (8 * i);
		p1 |= (u32)(d1 & 255) << (8 * i);
		p2 |= (u32)(d2 & 255) << (8 * i);
		s0 += d0;
		s1 += d1;
		s2 += d2;
	}
#pragma unroll
	for (int o = 1; o < 8; o <<= 1) {
		s0 += __shfl_xor(s0, o, 8);
		s1 += __shfl_xor(s1, o, 8);
		s2 += __shfl_xor(s2, o, 8);
	}
	dst[sub] = p2;
	dst[8 + sub] = p1;
	dst[16 + sub] = p0;
	if (sub == 0) {
		dst[24] = (u32)(127 - sh) << 23; /* 2^-s */
		dst[25] = (u32)s2;
		dst[26] = (u32)s1;
		dst[27] = (u32)s0;
	}
}

/* n floats (a multiple of 32) into staged digit blocks */
template <int NT>
__device__ static inline void stage_digits(u32 *dst, const float *src, int n)
{
	const float4 *s4 = (const float4 *)src;
	for (int i = threadIdx.x; i < n / 4; i += NT)
		stage_digits4(dst + (i / 8) * DBLK, s4[i], i & 7);
}

/* the same from a token held transposed in LDS: element k at
 * src[(k % 8) * RS + k / 8]; NTH threads, this one numbered tid (NTH a
 * multiple of 8: a block's 8 staging lanes are consecutive lanes of a wave) */
template <int NTH>
__device__ static inline void stage_digits_lds(u32 *dst, const float *src, int n, int RS,
					       int tid)
{
	for (int i = tid; i < n / 4; i += NTH) {
		const int r = (4 * i) & 7, c = (4 * i) >> 3;
		const float4 v = {src[r * RS + c], src[(r + 1) * RS + c], src[(r + 2) * RS + c],
				  src[(r + 3) * RS + c]};
		stage_digits4(dst + (i / 8) * DBLK, v, i & 7);
	}
}

/* sum_k q_k v_k of one block: q as 8 dwords of signed bytes (Q8_0) */
__device__ static inline float idot_q8(const u32 (&q)[8], const u32 *x)
{
	int S2 = 0, S1 = 0, S0 = 0;
#pragma unroll
	for (int k = 0; k < 8; k++) {
		S2 = __builtin_amdgcn_sdot4((int)q[k], (int)x[k], S2, false);
		S1 = __builtin_amdgcn_sdot4((int)q[k], (int)x[8 + k], S1, false);
		S0 = __builtin_amdgcn_sdot4((int)q[k], (int)x[16 + k], S0, false);
	}
	return ((float)S2 * 65536.0f + (float)(S1 * 256 + S0)) * __builtin_bit_cast(float, x[24]);
}

/* the same for Q4_0: 4 dwords of packed nibbles n = q + 8 (byte j: element
 * j low, j + 16 high) */
__device__ static inline float idot_q4(const u32 (&w)[4], const u32 *x)
{
	int S2 = 0, S1 = 0, S0 = 0;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		const int lo = (int)(w[k] & 0x0f0f0f0fu), hi = (int)((w[k] >> 4) & 0x0f0f0f0fu);
		S2 = __builtin_amdgcn_sdot4(lo, (int)x[k], S2, false);
		S2 = __builtin_amdgcn_sdot4(hi, (int)x[4 + k], S2, false);
		S1 = __builtin_amdgcn_sdot4(lo, (int)x[8 + k], S1, false);
		S1 = __builtin_amdgcn_sdot4(hi, (int)x[12 + k], S1, false);
		S0 = __builtin_amdgcn_sdot4(lo, (int)x[16 + k], S0, false);
		S0 = __builtin_amdgcn_sdot4(hi, (int)x[20 + k], S0, false);
	}
	S2 -= 8 * (int)x[25];
	S1 -= 8 * (int)x[26];
	S0 -= 8 * (int)x[27];
	return ((float)S2 * 65536.0f + (float)(S1 * 256 + S0)) * __builtin_bit_cast(float, x[24]);
}

/* a lane's gate/up segment against staged digits: Q8_0 one block (window
 * parity = block parity), Q4_0 a pair of blocks */
template <int WT> struct idig;
template <> struct idig<1> {
	static constexpr int NB = 1;
	__device__ static inline float dot(const u32 (&d)[9], const u32 *x, int s)
	{
		u32 q[8];
		const bool odd = s & 1;
#pragma unroll
		for (int k = 0; k < 8; k++)
			q[k] = odd ? d[k + 1] : __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		return f16_bits_to_f32(odd ? d[0] >> 16 : d[0]) * idot_q8(q, x);
	}
};
template <> struct idig<2> {
	static constexpr int NB = 2;
	__device__ static inline float dot(const u32 (&d)[9], const u32 *x, int)
	{
		u32 q0[4], q1[4];
#pragma unroll
		for (int k = 0; k < 4; k++) {
			q0[k] = __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
			q1[k] = d[5 + k];
		}
		return f16_bits_to_f32(d[0]) * idot_q4(q0, x) +
		       f16_bits_to_f32(d[4] >> 16) * idot_q4(q1, x + DBLK);
	}
};

/* a down-panel block (row i) against the item's h digits */
template <int WT> struct pdig;
template <> struct pdig<1> {
	__device__ static inline float dot(const u32 (&d)[9], int i, const u32 *h)
	{
		return idig<1>::dot(d, h, i);
	}
};
template <> struct pdig<2> {
	__device__ static inline float dot(const u32 (&d)[5], int i, const u32 *h)
	{
		u32 q[4];
		const bool odd = i & 1;
#pragma unroll
		for (int k = 0; k < 4; k++)
			q[k] = odd ? d[k + 1] : __builtin_amdgcn_alignbit(d[k + 1], d[k], 16);
		return f16_bits_to_f32(odd ? d[0] >> 16 : d[0]) * idot_q4(q, h);
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
template <int NT, int COLS>
__device__ static inline void stage_seg(float *s, const float *g, int n)
{
	const float4 *g4 = (const float4 *)g;
	for (int i = threadIdx.x; i < n / 4; i += NT) {
		int k = 4 * i;
		*(float4 *)(s + (k / COLS) * (COLS + 4) + k % COLS) = g4[i];
	}
}

/* ---------------------------------------------------------------------- */
/* routing                                                                */
/* ---------------------------------------------------------------------- */

/* copy n floats, element k -> dst[(k & 7) * RS + (k >> 3)] */
template <int NT>
__device__ static inline void stage_transposed(float *dst, const float *src, int n, int RS)
{
	const float4 *s4 = (const float4 *)src;
	for (int i = threadIdx.x; i < n / 4; i += NT) {
		float4 v = s4[i];
		int k = 4 * i;
		dst[((k + 0) & 7) * RS + ((k + 0) >> 3)] = v.x;
		dst[((k + 1) & 7) * RS + ((k + 1) >> 3)] = v.y;
		dst[((k + 2) & 7) * RS + ((k + 2) >> 3)] = v.z;
		dst[((k + 3) & 7) * RS + ((k + 3) >> 3)] = v.w;
	}
}

/* acc = fma(x[k], w[k], acc) over k = 0, 8, 16, ... of one transposed row
 * pair (E8 floats each).  The chain is 256 dependent FMAs for E = 2048; its
 * LDS operands come in batches of 8 FMAs (4 reads), four batches in
 * rotation, each loaded three batches ahead of its FMAs (12 reads in
 * flight: the LDS counter, 4 bits, can wait for exactly the oldest). */
struct chain_batch {
	float4 x[2], w[2];
	__device__ inline void load(const float4 *xr, const float4 *wr, int b)
	{
#pragma unroll
		for (int u = 0; u < 2; u++) {
			x[u] = xr[2 * b + u];
			w[u] = wr[2 * b + u];
		}
	}
	__device__ inline float run(float acc) const
	{
#pragma unroll
		for (int u = 0; u < 2; u++) {
			acc = __builtin_fmaf(x[u].x, w[u].x, acc);
			acc = __builtin_fmaf(x[u].y, w[u].y, acc);
			acc = __builtin_fmaf(x[u].z, w[u].z, acc);
			acc = __builtin_fmaf(x[u].w, w[u].w, acc);
		}
		return acc;
	}
};

/* NB (batches) a multiple of 4: the loop has no early exit, which keeps
 * the compiler's LDS waits at "all but the two younger batches" (an exit
 * inside the loop made them wait for every read: 12.8 -> 10.2 clocks per
 * FMA measured alone).  The loads run up to 3 batches (24 floats) past a
 * row's E8: the rows are followed by RS - E8 = 4 floats of padding and the
 * staging area by CHAIN_OVERRUN floats. */
#define CHAIN_OVERRUN 64
__device__ static inline float router_chain(const float *xrow, const float *wrow, int NB)
{
	const float4 *xr = (const float4 *)xrow, *wr = (const float4 *)wrow;
	chain_batch A, B, C, D;
	float acc = 0.0f;
	/* the scheduling barriers keep each batch's reads where they are
	 * issued: three batches ahead of their FMAs */
	A.load(xr, wr, 0);
	B.load(xr, wr, 1);
	C.load(xr, wr, 2);
	__builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
	for (int b = 0; b < NB; b += 4) {
		D.load(xr, wr, b + 3);
		__builtin_amdgcn_sched_barrier(0);
		acc = A.run(acc);
		__builtin_amdgcn_sched_barrier(0);
		A.load(xr, wr, b + 4);
		__builtin_amdgcn_sched_barrier(0);
		acc = B.run(acc);
		__builtin_amdgcn_sched_barrier(0);
		B.load(xr, wr, b + 5);
		__builtin_amdgcn_sched_barrier(0);
		acc = C.run(acc);
		__builtin_amdgcn_sched_barrier(0);
		C.load(xr, wr, b + 6);
		__builtin_amdgcn_sched_barrier(0);
		acc = D.run(acc);
		__builtin_amdgcn_sched_barrier(0);
	}
	return acc;
}

/*
 * One token's rms_norm(h) * w in every workgroup of a NORM launch.  The rms
 * is taken as the one-token model kernels take it, with 256 threads whose
 * sums go through xor trees in waves of 64 and then the four waves' sums
 * in order, sqrtf(sum / E + 1e-5f): ORD 1 as the output product's gathered
 * norm (thread v adds h[v]^2, h[v + 256]^2, ... in order), ORD 2 as the
 * row norm kernel's (thread v adds the four squares of float4 v, then of
 * float4 v + 256, ...).  So every workgroup, and the norm launch it
 * replaces, get the same bits; then x = (h / rms) * w (olmoe.c:486-488,
 * rmsnorm nn.c:8-31).  hv: this thread's float4s i = tid + NT v (< E / 4)
 * of the token, normalised.  The whole workgroup calls it.
 */
template <int NT, int NV, int ORD>
__device__ static void norm_token(const float *h, const float *w, int E, float4 (&hv)[NV])
{
	static_assert(ORD == 1 || ORD == 2, "a summation order");
	constexpr int MS = NV * NT / 64; /* ORD 1: terms of a summing thread (E / 256) */
	constexpr int M4 = NV * NT / 256; /* ORD 2: its float4s (E / 1024) */
	__shared__ float s_red[4];
	const float4 *h4 = (const float4 *)h, *w4 = (const float4 *)w;
	const int tid = threadIdx.x, lane = tid % WAVE;
	float4 wv[NV];
#pragma unroll
	for (int v = 0; v < NV; v++) {
		const int i = tid + NT * v;
		if (i < E / 4) {
			hv[v] = h4[i];
			wv[v] = w4[i];
		}
	}
	float ss = 0.0f;
	if (tid < 256) {
		if constexpr (ORD == 1) {
			float sv[MS];
#pragma unroll
			for (int m = 0; m < MS; m++)
				sv[m] = 256 * m + tid < E ? h[256 * m + tid] : 0.0f;
#pragma unroll
			for (int m = 0; m < MS; m++)
				if (256 * m + tid < E) {
					const float t = sv[m] * sv[m];
					ss = ss + t;
				}
		} else {
			float4 sv[M4 > 0 ? M4 : 1];
#pragma unroll
			for (int m = 0; m < (M4 > 0 ? M4 : 1); m++)
				if (256 * m + tid < E / 4)
					sv[m] = h4[256 * m + tid];
#pragma unroll
			for (int m = 0; m < (M4 > 0 ? M4 : 1); m++)
				if (256 * m + tid < E / 4) {
					const float q0 = sv[m].x * sv[m].x, q1 = sv[m].y * sv[m].y;
					const float q2 = sv[m].z * sv[m].z, q3 = sv[m].w * sv[m].w;
					ss = ss + q0;
					ss = ss + q1;
					ss = ss + q2;
					ss = ss + q3;
				}
		}
		for (int o = WAVE / 2; o > 0; o >>= 1)
			ss += __shfl_xor(ss, o, WAVE);
		if (lane == 0)
			s_red[tid / WAVE] = ss;
	}
	__syncthreads();
	float sum = 0.0f;
#pragma unroll
	for (int k = 0; k < 4; k++)
		sum += s_red[k];
	const float rms = sqrtf(sum / (float)E + 1e-5f);
#pragma unroll
	for (int v = 0; v < NV; v++)
		if (tid + NT * v < E / 4) {
			float r = hv[v].x / rms;
			hv[v].x = r * wv[v].x;
			r = hv[v].y / rms;
			hv[v].y = r * wv[v].y;
			r = hv[v].z / rms;
			hv[v].z = r * wv[v].z;
			r = hv[v].w / rms;
			hv[v].w = r * wv[v].w;
		}
}

/* router row j for every token, published into every replica by wave 0;
 * prev_epoch (the launch's epoch minus one, valid in thread 0) is consumed
 * only after the chain, so its load is in flight meanwhile.  dig (one
 * token): the other waves stage the token's digit blocks there while wave
 * 0 runs the chain. */
template <int NT, int E, int NORM = 0>
__device__ static void router_row(const DecodeArgs &a, int j, u32 prev_epoch, float *lds,
				  u32 *dig)
{
	static_assert(E % 256 == 0, "the chain runs whole rounds of four batches");
	constexpr int E8 = E / 8, RS = E8 + 4;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	float *sw = lds;          /* [8][RS] router row, transposed */
	float *sx = lds + 8 * RS; /* [8][RS] token, transposed */
	__shared__ float s_logit;
	uint64_t *rep = (uint64_t *)(a.sync + a.off_rep);

	if (a.T == 1) {
		/* one token: the row and the token arrive in one round trip and
		 * land transposed in LDS (element k at [k % 8][k / 8]); then the
		 * chains run from registers.  Lane 8c + s of wave 0 reads elements
		 * 8m + c for m in segment s (M = E / 64 of them, contiguous in the
		 * transposed copy) and runs that stretch of AVX2 lane c's chain;
		 * segment s + 1 takes the running sum from lane 8c + s (a DPP shift
		 * inside the lanes' 16-lane row), so each chain keeps its FMAs and
		 * their order.  The other waves stage the token's digit blocks
		 * from the LDS copy meanwhile. */
		constexpr int M = E / 64;
		const float4 *w4 = (const float4 *)(a.router + (size_t)j * E);
		const float4 *x4 = (const float4 *)a.x;
		auto put = [&](int i, float4 wv, float4 xv) {
			const int k = 4 * i;
			sw[((k + 0) & 7) * RS + ((k + 0) >> 3)] = wv.x;
			sw[((k + 1) & 7) * RS + ((k + 1) >> 3)] = wv.y;
			sw[((k + 2) & 7) * RS + ((k + 2) >> 3)] = wv.z;
			sw[((k + 3) & 7) * RS + ((k + 3) >> 3)] = wv.w;
			sx[((k + 0) & 7) * RS + ((k + 0) >> 3)] = xv.x;
			sx[((k + 1) & 7) * RS + ((k + 1) >> 3)] = xv.y;
			sx[((k + 2) & 7) * RS + ((k + 2) >> 3)] = xv.z;
			sx[((k + 3) & 7) * RS + ((k + 3) >> 3)] = xv.w;
		};
		if constexpr (NORM != 0) {
			/* the row's loads go out with the residual's and the norm
			 * weights'; x = rms_norm(h) * w lands in LDS (and x_out) */
			constexpr int NV = (E / 4 + NT - 1) / NT;
			float4 rv[NV], hv[NV];
#pragma unroll
			for (int v = 0; v < NV; v++)
				if ((int)threadIdx.x + NT * v < E / 4)
					rv[v] = w4[threadIdx.x + NT * v];
			norm_token<NT, NV, NORM>(a.x, a.norm_w, E, hv);
#pragma unroll
			for (int v = 0; v < NV; v++) {
				const int i = threadIdx.x + NT * v;
				if (i < E / 4) {
					put(i, rv[v], hv[v]);
					if (j == 0)
						((float4 *)a.x_out)[i] = hv[v];
				}
			}
		} else {
			for (int i = threadIdx.x; i < E / 4; i += NT)
				put(i, w4[i], x4[i]);
		}
		__syncthreads();
		if (wave == 0) {
			const int c = lane >> 3, sg = lane & 7;
			const float4 *wr = (const float4 *)(sw + c * RS + M * sg);
			const float4 *xr = (const float4 *)(sx + c * RS + M * sg);
			float4 wv[M / 4], xv[M / 4];
#pragma unroll
			for (int i = 0; i < M / 4; i++) {
				wv[i] = wr[i];
				xv[i] = xr[i];
			}
			float acc = 0.0f;
#pragma unroll
			for (int q = 0; q < 8; q++) {
				if (sg == q)
#pragma unroll
					for (int i = 0; i < M / 4; i++) {
						acc = __builtin_fmaf(xv[i].x, wv[i].x, acc);
						acc = __builtin_fmaf(xv[i].y, wv[i].y, acc);
						acc = __builtin_fmaf(xv[i].z, wv[i].z, acc);
						acc = __builtin_fmaf(xv[i].w, wv[i].w, acc);
					}
				if (q < 7) /* lane 8c + q + 1 <- lane 8c + q */
					acc = __builtin_bit_cast(
						float, __builtin_amdgcn_update_dpp(
							       0, __builtin_bit_cast(int, acc), 0x111, 0xf,
							       0xf, false));
			}
			/* chain c's sum sits in lane 8c + 7: lanes 0-7 take them, then
			 * the AVX2 tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
			acc = __shfl(acc, 8 * (lane & 7) + 7, WAVE);
			acc = acc + __shfl_xor(acc, 4, 8);
			acc = acc + __shfl_xor(acc, 2, 8);
			acc = acc + __shfl_xor(acc, 1, 8);
			if (lane == 0)
				s_logit = (a.bias ? a.bias[j] : 0.0f) + acc;
		} else if (dig) {
			stage_digits_lds<NT - WAVE>(dig, sx, E, RS, (int)threadIdx.x - WAVE);
		}
		__syncthreads();
		if (wave == 0) { /* NREP == WAVE: lane r writes replica r */
			const u32 ep = __shfl(prev_epoch, 0, WAVE) + 1;
			const uint64_t v = ((uint64_t)ep << 32) | __builtin_bit_cast(u32, s_logit);
			st_dev_u64(&rep[(size_t)lane * a.rep_stride + (size_t)j], v);
		}
		__syncthreads();
		return;
	}
	for (int t = 0; t < a.T; t++) {
		if (t == 0) { /* router row and token 0: one round trip */
			const float4 *w4 = (const float4 *)(a.router + (size_t)j * E);
			const float4 *x4 = (const float4 *)a.x;
			for (int i = threadIdx.x; i < E / 4; i += NT) {
				const float4 wv = w4[i], xv = x4[i];
				const int k = 4 * i;
				sw[((k + 0) & 7) * RS + ((k + 0) >> 3)] = wv.x;
				sw[((k + 1) & 7) * RS + ((k + 1) >> 3)] = wv.y;
				sw[((k + 2) & 7) * RS + ((k + 2) >> 3)] = wv.z;
				sw[((k + 3) & 7) * RS + ((k + 3) >> 3)] = wv.w;
				sx[((k + 0) & 7) * RS + ((k + 0) >> 3)] = xv.x;
				sx[((k + 1) & 7) * RS + ((k + 1) >> 3)] = xv.y;
				sx[((k + 2) & 7) * RS + ((k + 2) >> 3)] = xv.z;
				sx[((k + 3) & 7) * RS + ((k + 3) >> 3)] = xv.w;
			}
		} else {
			stage_transposed<NT>(sx, a.x + (size_t)t * E, E, RS);
		}
		__syncthreads();
		if (wave == 0) {
			/* lane l < 8 replays AVX2 lane l: elements l, l+8, ... in order */
			const int l = lane & 7;
			float acc = router_chain(sx + l * RS, sw + l * RS, a.E / 64);
			acc = acc + __shfl_xor(acc, 4, 8);
			acc = acc + __shfl_xor(acc, 2, 8);
			acc = acc + __shfl_xor(acc, 1, 8);
			if (lane == 0)
				s_logit = (a.bias ? a.bias[j] : 0.0f) + acc;
		} else if (t == 0 && dig) {
			stage_digits_lds<NT - WAVE>(dig, sx, E, RS, (int)threadIdx.x - WAVE);
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
 * w, w + NT/64, ...; lane j polls entry (t, j) until the whole row carries
 * the epoch (one hop: the loads that see the epoch also deliver the
 * logits), then the wave runs softmax + top-k (+ renorm) into s_ids/s_w
 * [T*K].
 */
template <int NT>
__device__ static void route_local(const DecodeArgs &a, u32 epoch, float *lds, u32 *s_ids,
				   float *s_w, const uint64_t *s_tab)
{
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const uint64_t *rep = (const uint64_t *)(a.sync + a.off_rep) +
			      (size_t)(blockIdx.x % NREP) * a.rep_stride;
	float *scr = lds + wave * (MOE_MAX_NE + 2 * MOE_MAX_TOPK);
	if (a.T == 1) {
		/* one token: wave 0 polls and runs the softmax; every wave ranks
		 * each key against 64 / NW of the others; wave 0 adds the parts
		 * and fills the slots */
		constexpr int NW = NT / WAVE, PER = WAVE / NW;
		static_assert(PER % 2 == 0, "keys are read in pairs");
		__shared__ __attribute__((aligned(16))) uint64_t s_key[WAVE];
		__shared__ int s_rk[NW][WAVE];
		float p = 0.0f;
		if (wave == 0) {
			const uint64_t idle = (uint64_t)epoch << 32;
			uint64_t v = 0;
			int step = 0;
			for (int round = 0;; round++) {
				v = lane < a.NE ? ld_dev_u64(&rep[lane]) : idle;
				if (__all((u32)(v >> 32) == epoch))
					break;
				if (round >= a.spin) {
					if (lane == 0)
						st_dev_u32(a.sync + MOE_SYNC_ERR_WORD, MOE_ERR_ROUTE);
					break;
				}
				backoff(step);
			}
			uint64_t key;
			p = softmax64(__builtin_bit_cast(float, (u32)v), a.NE, s_tab, lane, key);
			s_key[lane] = key;
		}
		__syncthreads();
		s_rk[wave][lane] = rank_part64(s_key + wave * PER, PER, s_key[lane]);
		__syncthreads();
		if (wave == 0) {
			int rank = 0;
#pragma unroll
			for (int w = 0; w < NW; w++)
				rank += s_rk[w][lane];
			topk_finish64(rank, p, s_ids, s_w, a.NE, a.K, a.renorm,
				      (u32 *)(scr + MOE_MAX_NE), scr + MOE_MAX_NE + MOE_MAX_TOPK, lane);
		}
		__syncthreads();
		return;
	}
	for (int t = wave; t < a.T; t += NT / WAVE) { /* NE <= 64: one expert per lane */
		const uint64_t *row = rep + (size_t)t * a.NE;
		float logit = 0.0f;
		int step = 0;
		for (int round = 0;; round++) {
			const uint64_t v = lane < a.NE ? ld_dev_u64(&row[lane]) : (uint64_t)epoch << 32;
			if (__all((u32)(v >> 32) == epoch)) {
				logit = __builtin_bit_cast(float, (u32)v);
				break;
			}
			if (round >= a.spin) {
				if (lane == 0)
					st_dev_u32(a.sync + MOE_SYNC_ERR_WORD, MOE_ERR_ROUTE);
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
/* items                                                                  */
/* ---------------------------------------------------------------------- */

template <int WT, int CG, int NT> struct gu_geo {
	static constexpr int NW = NT / WAVE;
	static constexpr int HR = DEC_CHUNK / NW; /* h rows per wave */
	static constexpr int RPS = WAVE / CG;     /* rows per wave step */
	static constexpr int NS = HR / RPS;       /* wave steps per item */
	static_assert(NS >= 1 && NS * RPS == HR, "a wave's rows must fill its steps");
};

/* an item's weights in registers: gate and up windows, down panel blocks */
template <int WT, int CG, int NT, int RPT> struct item_regs {
	u32 g[gu_geo<WT, CG, NT>::NS][segq<WT>::DW];
	u32 u[gu_geo<WT, CG, NT>::NS][segq<WT>::DW];
	u32 d[RPT][panel_blk<WT>::DW];
};

template <int WT, int CG, int NT, int RPT>
__device__ static inline void load_gateup(const DecodeArgs &a, int q, const u32 *s_ids,
					  item_regs<WT, CG, NT, RPT> &r, bool active)
{
	if (!active)
		return;
	typedef segq<WT> S;
	typedef gu_geo<WT, CG, NT> GG;
	const int NC = a.EI / DEC_CHUNK, p = q / NC, c = q % NC;
	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int seg = lane % CG, sub = lane / CG;
	const size_t rb = (size_t)(a.E / MOE_QK) * (WT == 1 ? 34 : 18);
	const size_t eo = (size_t)s_ids[p] * a.gu_stride;
	const uint8_t *G = S::win(a.gate + eo, seg), *U = S::win(a.up + eo, seg);
#pragma unroll
	for (int s2 = 0; s2 < GG::NS; s2++) {
		const size_t ro =
			(size_t)(c * DEC_CHUNK + wave * GG::HR + s2 * GG::RPS + sub) * rb;
		load_dwords<S::DW>(G + ro, r.g[s2]);
		load_dwords<S::DW>(U + ro, r.u[s2]);
	}
}

template <int WT, int CG, int NT, int RPT>
__device__ static inline void load_down(const DecodeArgs &a, int q, const u32 *s_ids,
					item_regs<WT, CG, NT, RPT> &r)
{
	typedef panel_blk<WT> D;
	const int NC = a.EI / DEC_CHUNK, p = q / NC, c = q % NC;
	const uint8_t *panel =
		a.down + (size_t)s_ids[p] * a.dn_stride + (size_t)c * a.E * D::BB;
#pragma unroll
	for (int r2 = 0; r2 < RPT; r2++) {
		const int i = threadIdx.x + NT * r2;
		load_dwords<D::DW>(panel + ((D::BB * i) & ~3), r.d[r2]);
	}
}

/*
 * WT: 1 = Q8_0, 2 = Q4_0.  CG: lanes per gate/up row (E / segment columns).
 * NT: threads (one workgroup per CU).  RPT = E / NT: down rows per thread.
 */
template <int WT, int CG, int NT, int RPT, bool NORM>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT / 256, NT / 256)))
void k_moe_decode(DecodeArgs a)
{
	typedef segq<WT> S;
	typedef panel_blk<WT> D;
	typedef gu_geo<WT, CG, NT> GG;
	extern __shared__ float lds[];
	__shared__ u32 s_ids[MOE_FUSED_MAX_P];
	__shared__ float s_w[MOE_FUSED_MAX_P];
	__shared__ u32 s_epoch;
	__shared__ u32 s_poison;
	__shared__ uint64_t s_tab[32];
	__shared__ __attribute__((aligned(16))) float s_h[DEC_CHUNK];
	__shared__ __attribute__((aligned(16))) u32 s_hd[NT / WAVE][DBLK];
	__shared__ int s_ok;

	const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
	const int G = (int)gridDim.x, b = (int)blockIdx.x;
	const int NC = a.EI / DEC_CHUNK, IPT = a.K * NC, N = a.n_items;
	STAMP(0);
	/* work is dealt in half items (16 rows of d_ff), so that every
	 * workgroup gets the same share when the items do not divide evenly
	 * (Mixtral: 3.5 items each); x0 .. x1 are this workgroup's halves */
	const int N2 = 2 * N;
	const int x0 = item_lo(b, N2, G), x1 = item_lo(b + 1, N2, G);
	const int t0 = x0 / 2 / IPT;
	const int XS = (a.E / MOE_QK) * DBLK;           /* dwords of one staged token */
	u32 *sx = (u32 *)lds;                           /* [DEC_TOKS][XS] token digits */
	float *rl = lds + DEC_TOKS * XS;                /* routing scratch */

	if (threadIdx.x < 32)
		s_tab[threadIdx.x] = moe_exp2_tab[threadIdx.x];
	u32 prev_epoch = 0, err0 = 0;
	if (threadIdx.x == 0) { /* consumed late: the loads overlap routing */
		prev_epoch = ld_dev_u32(a.sync);
		err0 = ld_dev_u32(a.sync + MOE_SYNC_ERR_WORD);
	}
	/* one token: a router workgroup stages it from its router row's LDS
	 * copy (no second round trip) */
	const bool st0 = b < a.NE && x0 < x1 && a.T == 1;
	if (b < a.NE)
		router_row<NT, CG * S::COLS, NORM ? 1 : 0>(a, b, prev_epoch, rl, st0 ? sx : nullptr);
	/* the tokens of this workgroup's items (they do not depend on routing) */
	if (x0 < x1 && !st0) {
		if constexpr (NORM) { /* one token, normalised here */
			constexpr int NV = (RPT + 3) / 4;
			float4 hv[NV];
			norm_token<NT, NV, 1>(a.x, a.norm_w, a.E, hv);
#pragma unroll
			for (int v = 0; v < NV; v++) {
				const int i = threadIdx.x + NT * v;
				if (i < a.E / 4)
					stage_digits4(sx + (i / 8) * DBLK, hv[v], i & 7);
			}
		} else {
			for (int t = t0; t <= (x1 - 1) / 2 / IPT; t++)
				stage_digits<NT>(sx + (t - t0) * XS, a.x + (size_t)t * a.E, a.E);
		}
	}
	if (threadIdx.x == 0) {
		s_epoch = prev_epoch + 1;
		s_poison = err0;
	}
	__syncthreads();
	const u32 epoch = s_epoch;
	/* a wait of an earlier launch ran out: the flags, replicas and partials
	 * may hold tags this epoch would accept, so every launch until the host
	 * clears the sync words (hip_moe_status) writes NaN outputs and returns
	 * without raising its start flag or advancing the epoch */
	if (s_poison) {
		const float nan = __builtin_nanf("");
		for (int i = b * NT + (int)threadIdx.x; i < a.T * a.E; i += G * NT)
			a.out[i] = nan;
		if (b == 0)
			for (int i = threadIdx.x; i < a.T * a.K; i += NT) {
				a.ids_out[i] = 0;
				a.w_out[i] = nan;
			}
		return;
	}
	/* this workgroup has read the epoch word: workgroup 0 may advance it
	 * once every workgroup has said so */
	u32 *startf = a.sync + a.off_start;
	if (threadIdx.x == 0 && b != 0)
		st_dev_u32(&startf[b], epoch);
	route_local<NT>(a, epoch, rl, s_ids, s_w, s_tab);
	STAMP(1);
	if (b == 0)
		for (int i = threadIdx.x; i < a.T * a.K; i += NT) {
			a.ids_out[i] = s_ids[i];
			a.w_out[i] = s_w[i];
		}

	/* ---- items ---- */
	const int seg = lane % CG, sub = lane / CG;
	float acc[RPT];
#pragma unroll
	for (int r2 = 0; r2 < RPT; r2++)
		acc[r2] = 0.0f;
	item_regs<WT, CG, NT, RPT> R;

	/* h rows of this wave: silu(gate . x) * (up . x), or zeros when the
	 * unit is the other half of the item */
	auto gateup = [&](int q, bool active) {
		if (!active) {
			if (seg == 0)
#pragma unroll
				for (int s2 = 0; s2 < GG::NS; s2++)
					s_h[wave * GG::HR + s2 * GG::RPS + sub] = 0.0f;
			return;
		}
		const int t = q / NC / a.K;
		typedef idig<WT> I;
		u32 xd[I::NB * DBLK]; /* this lane's segment: NB staged blocks */
		{
			const uint4 *s4 = (const uint4 *)(sx + (t - t0) * XS + seg * I::NB * DBLK);
#pragma unroll
			for (int k = 0; k < I::NB * DBLK / 4; k++) {
				const uint4 v = s4[k];
				xd[4 * k + 0] = v.x;
				xd[4 * k + 1] = v.y;
				xd[4 * k + 2] = v.z;
				xd[4 * k + 3] = v.w;
			}
		}
#pragma unroll
		for (int s2 = 0; s2 < GG::NS; s2++) {
			const float gv = group_sum<CG>(I::dot(R.g[s2], xd, seg));
			const float uv = group_sum<CG>(I::dot(R.u[s2], xd, seg));
			if (seg == 0)
				s_h[wave * GG::HR + s2 * GG::RPS + sub] =
					(gv / (1.0f + moe_expf_tab(-gv, s_tab))) * uv;
		}
	};
	/* this item's share of every output row: down panel . h, scaled */
	auto down = [&](int q) {
		/* every wave turns the 32 h values into digits itself (lanes 0-31,
		 * its own LDS copy): no second workgroup barrier */
		u32 *hw = s_hd[wave];
		if (lane < DEC_CHUNK / 4)
			stage_digits4(hw, ((const float4 *)s_h)[lane], lane);
		WAVE_SYNC();
		u32 hd[DBLK];
		{
			const uint4 *s4 = (const uint4 *)hw;
#pragma unroll
			for (int k = 0; k < DBLK / 4; k++) {
				const uint4 v = s4[k];
				hd[4 * k + 0] = v.x;
				hd[4 * k + 1] = v.y;
				hd[4 * k + 2] = v.z;
				hd[4 * k + 3] = v.w;
			}
		}
		const float inv = 1.0f / s_w[q / NC];
#pragma unroll
		for (int r2 = 0; r2 < RPT; r2++)
			acc[r2] = acc[r2] +
				  pdig<WT>::dot(R.d[r2], (int)threadIdx.x + NT * r2, hd) / inv;
	};
	/* publish token t's accumulated outputs */
	auto flush = [&](int t) {
		const int con = b - item_owner(2 * t * IPT, N2, G);
		uint64_t *pt = a.part + (size_t)t * a.E * a.ncon;
#pragma unroll
		for (int r2 = 0; r2 < RPT; r2++) {
			const int i = threadIdx.x + NT * r2;
			st_dev_u64(&pt[((size_t)(i / PSLICE) * a.ncon + con) * PSLICE + i % PSLICE],
				   ((uint64_t)epoch << 32) | __builtin_bit_cast(u32, acc[r2]));
			acc[r2] = 0.0f;
		}
	};

	/* the units of [x0, x1): the second half of item x0 / 2 when x0 is odd,
	 * whole items, the first half of item x1 / 2 when x1 is odd.  A half
	 * streams its 16 gate/up rows (the other waves' h rows are zero) and
	 * the whole down panel. */
	const int head = x0 & 1, full0 = (x0 + 1) / 2, nfull = x1 / 2 - full0;
	const int nu = x0 < x1 ? head + nfull + (x1 & 1) : 0;
	auto unit = [&](int u, int &m) -> int { /* item; m: bit h = rows 16h .. 16h+15 */
		if (head && u == 0) {
			m = 2;
			return x0 / 2;
		}
		const int k = u - head;
		m = k < nfull ? 3 : 1;
		return k < nfull ? full0 + k : x1 / 2;
	};
	const int hw = wave / (NT / WAVE / 2); /* the half of the item's rows this wave holds */
	if (nu > 0) {
		int m, mn;
		int q = unit(0, m);
		load_gateup<WT, CG, NT, RPT>(a, q, s_ids, R, (m >> hw) & 1);
		load_down<WT, CG, NT, RPT>(a, q, s_ids, R);
		/* units before the last: the next unit's loads go into R right
		 * after the last reads of each part of it (the scheduling barriers
		 * keep them there, so R needs no copies and no waits at the loop's
		 * end) */
		for (int u = 0; u + 1 < nu; u++) {
			const int qn = unit(u + 1, mn);
			gateup(q, (m >> hw) & 1);
			__builtin_amdgcn_sched_barrier(0);
			load_gateup<WT, CG, NT, RPT>(a, qn, s_ids, R, (mn >> hw) & 1);
			__syncthreads(); /* s_h complete */
			down(q);
			__builtin_amdgcn_sched_barrier(0);
			load_down<WT, CG, NT, RPT>(a, qn, s_ids, R);
			if (qn / IPT != q / IPT)
				flush(q / IPT);
			__syncthreads(); /* s_h is rewritten next */
			q = qn;
			m = mn;
		}
		gateup(q, (m >> hw) & 1);
		__syncthreads();
		STAMP(2);
		down(q);
		flush(q / IPT);
		STAMP(3);
	}

	/* ---- combine: slices b, b + G, ... of the T*E outputs, NP at a time
	 * (two where a token's E outputs give each workgroup two or more
	 * slices, E = 4096: polled together; Mixtral T=1 58.1 -> 56.5 us) ----
	 * thread tid takes the entries e = tid + NT*k of a slice (contributor
	 * e / PSLICE, output e % PSLICE = tid % PSLICE) and adds them in k order;
	 * lanes of one output meet in an xor tree, waves in wave order */
	float *sc = lds; /* [NT / WAVE][NP][PSLICE] */
	const int NSL = a.E / PSLICE, NS_ALL = a.T * NSL;
	{
		constexpr int NP = RPT >= 8 ? 2 : 1; /* slices per workgroup and token: RPT / 4 */
		constexpr int KH = CMB_MAX / NP; /* entries per thread and slice */
		for (int sl0 = b; sl0 < NS_ALL; sl0 += NP * G) {
			const uint64_t *src[NP];
			unsigned pending = 0;
#pragma unroll
			for (int hs = 0; hs < NP; hs++) {
				const int sl = sl0 + hs * G;
				src[hs] = a.part + (size_t)min(sl, NS_ALL - 1) * a.ncon * PSLICE;
				if (sl >= NS_ALL)
					continue;
				const int t = sl / NSL;
				const int bf = item_owner(2 * t * IPT, N2, G),
					  bl = item_owner(2 * (t + 1) * IPT - 1, N2, G);
				const int n = (bl - bf + 1) * PSLICE;
				/* this thread's entries (at most KH), skipping workgroups
				 * without items */
#pragma unroll
				for (int k = 0; k < KH; k++) {
					const int e = threadIdx.x + NT * k, wb = bf + e / PSLICE;
					if (e < n && item_lo(wb, N2, G) != item_lo(wb + 1, N2, G))
						pending |= 1u << (hs * KH + k);
				}
			}
			/* each thread polls its own entries until their tags show the
			 * epoch, with no workgroup barrier per poll */
			const unsigned live = pending;
			float vals[CMB_MAX];
			for (int round = 0; pending; round++) {
				/* every pending load is issued before any is checked: one
				 * round trip per round, not one per entry */
				uint64_t v[CMB_MAX];
#pragma unroll
				for (int k = 0; k < CMB_MAX; k++)
					v[k] = (pending >> k) & 1u
						       ? ld_dev_u64(&src[k / KH][threadIdx.x + NT * (k % KH)])
						       : 0;
#pragma unroll
				for (int k = 0; k < CMB_MAX; k++)
					if ((pending >> k) & 1u) {
						vals[k] = __builtin_bit_cast(float, (u32)v[k]);
						if ((u32)(v[k] >> 32) == epoch)
							pending &= ~(1u << k);
					}
				if (!pending)
					break;
				if (round >= a.spin) {
					st_dev_u32(a.sync + MOE_SYNC_ERR_WORD, MOE_ERR_COMBINE);
					break;
				}
				__builtin_amdgcn_s_sleep(1);
			}
#pragma unroll
			for (int hs = 0; hs < NP; hs++) {
				float sum = 0.0f;
#pragma unroll
				for (int k = 0; k < KH; k++)
					if ((live >> (hs * KH + k)) & 1u)
						sum += vals[hs * KH + k];
				sum += __shfl_xor(sum, 8, WAVE);
				sum += __shfl_xor(sum, 16, WAVE);
				sum += __shfl_xor(sum, 32, WAVE);
				if (lane < PSLICE)
					sc[(wave * NP + hs) * PSLICE + lane] = sum;
			}
			__syncthreads();
			if (threadIdx.x < NP * PSLICE) {
				const int hs = threadIdx.x / PSLICE, sl = sl0 + hs * G;
				if (sl < NS_ALL) {
					float o = 0.0f;
					for (int w = 0; w < NT / WAVE; w++)
						o += sc[(w * NP + hs) * PSLICE + threadIdx.x % PSLICE];
					a.out[(size_t)(sl / NSL) * a.E + (sl % NSL) * PSLICE +
					      threadIdx.x % PSLICE] = o;
				}
			}
			__syncthreads();
		}
	}

	STAMP(4);
	/* workgroup 0 advances the epoch for the next launch once every
	 * workgroup has read it (they did so long ago: no wait in practice);
	 * the next launch starts only after this one drains */
	if (b != 0)
		return;
	/* a workgroup that has not started by now would read the advanced
	 * epoch and tag its data for the next launch: the epoch stays, and the
	 * error word (sticky) stops every launch until the host resets */
	if (wait_flags<NT>(startf + 1, G - 1, epoch, a.sync + MOE_SYNC_ERR_WORD, MOE_ERR_FLAGS,
			   a.spin) &&
	    threadIdx.x == 0)
		st_dev_u32(a.sync, epoch);
}

/* ---------------------------------------------------------------------- */

struct Geo {
	int NT, CG, RPT, cols;
	const void *fn, *fn_norm; /* x ready / x = rms_norm(h) * w in the launch */
};

/* 512 threads (two waves per SIMD: 256 VGPRs for an item's weights and
 * activations); Q8_0 32-column lane segments, Q4_0 64.  Instances cover
 * d_model 1024 and 2048 (Q8_0), 2048 and 4096 (Q4_0). */
static Geo geometry(int wtype, size_t E, size_t EI)
{
	Geo g;
	g.fn = g.fn_norm = NULL;
	g.cols = wtype == 1 ? 32 : 64;
	g.NT = 512;
	g.CG = (int)(E / (size_t)g.cols);
	g.RPT = (int)(E / (size_t)g.NT);
	if (E % (size_t)g.cols || E % (size_t)g.NT || EI % DEC_CHUNK || EI == 0)
		return g;
#define PICK(W_, CG_, NT_, RPT_)                                                    \
	if (wtype == W_ && g.CG == CG_ && g.NT == NT_ && g.RPT == RPT_) {            \
		g.fn = (const void *)k_moe_decode<W_, CG_, NT_, RPT_, false>;         \
		g.fn_norm = (const void *)k_moe_decode<W_, CG_, NT_, RPT_, true>;     \
	}
	PICK(1, 32, 512, 2)
	PICK(1, 64, 512, 4)
	PICK(2, 32, 512, 4)
	PICK(2, 64, 512, 8)
#undef PICK
	return g;
}

/* dynamic LDS: DEC_TOKS staged tokens + routing scratch (router row and
 * token transposed, or the per-wave top-k scratch); the combine reuses the
 * front (one PSLICE-float partial per wave) */
static size_t decode_lds_bytes(const Geo &g, size_t E)
{
	size_t xs = DEC_TOKS * (E / MOE_QK) * DBLK;
	size_t rt = (size_t)2 * 8 * (E / 8 + 4) + CHAIN_OVERRUN;
	size_t tk = (size_t)(g.NT / WAVE) * (MOE_MAX_NE + 2 * MOE_MAX_TOPK);
	return (xs + (rt > tk ? rt : tk)) * sizeof(float);
}

/* the largest number of workgroups holding items of one token */
static int decode_ncon(size_t T, size_t K, size_t EI, int grid)
{
	const int IPT = (int)(K * (EI / DEC_CHUNK)), N2 = 2 * (int)T * IPT; /* half items */
	int m = 1;
	for (int t = 0; t < (int)T; t++) {
		int c = item_owner(2 * (t + 1) * IPT - 1, N2, grid) - item_owner(2 * t * IPT, N2, grid) + 1;
		if (c > m)
			m = c;
	}
	return m;
}

struct SyncLayout {
	size_t off_start, off_rep, words, rep_stride;
};

static SyncLayout sync_layout(size_t T, size_t NE, int grid)
{
	SyncLayout s;
	s.rep_stride = (T * NE + 511) & ~(size_t)511;
	s.off_start = 1024;
	s.off_rep = s.off_start + (((size_t)grid + 1023) & ~(size_t)1023);
	s.words = s.off_rep + (size_t)NREP * s.rep_stride * 2;
	return s;
}

extern "C" int moe_fused_supported(int wtype, size_t E, size_t EI, size_t NE, size_t T,
				   size_t K)
{
	if (NE > WAVE || T * K > MOE_FUSED_MAX_P || T == 0 || E % 128)
		return 0;
	return geometry(wtype, E, EI).fn != NULL;
}

extern "C" size_t moe_fused_sync_words(size_t T, size_t NE, int grid)
{
	return sync_layout(T, NE, grid).words;
}

extern "C" size_t moe_fused_part_words(size_t T, size_t K, size_t E, size_t EI, int grid)
{
	return T * E * (size_t)decode_ncon(T, K, EI, grid);
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
	int per_n = 0;
	if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, g.fn, g.NT,
							 decode_lds_bytes(g, E)) != hipSuccess ||
	    per < 1 ||
	    hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_n, g.fn_norm, g.NT,
							 decode_lds_bytes(g, E)) != hipSuccess ||
	    per_n < 1)
		return 0;
	/* one workgroup per CU; the router rows need one workgroup each, a
	 * workgroup's items must span at most DEC_TOKS tokens (T <= grid), and
	 * a combine thread covers at most CMB_MAX / 2 entries of a slice */
	return ncu >= (int)NE && ncu >= MOE_FUSED_MAX_P && ncu * PSLICE <= CMB_MAX / 2 * g.NT
		       ? ncu
		       : 0;
}

extern "C" int moe_launch_fused(int wtype, const float *x, const float *router,
				const float *bias, const uint8_t *gate, const uint8_t *up,
				const uint8_t *down, size_t gu_stride, size_t dn_stride,
				uint32_t *ids, float *w, uint64_t *part, float *out, uint32_t *sync,
				int T, int E, int EI, int NE, int K, int renorm, int grid,
				int spin, const float *norm_w, float *x_out, void *stream)
{
	Geo g = geometry(wtype, (size_t)E, (size_t)EI);
	if (!g.fn || grid < NE || grid < T || (norm_w && (T != 1 || !x_out)))
		return (int)hipErrorInvalidValue;
	SyncLayout sl = sync_layout((size_t)T, (size_t)NE, grid);
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
	a.part = part;
	a.out = out;
	a.sync = sync;
	a.T = T;
	a.E = E;
	a.EI = EI;
	a.NE = NE;
	a.K = K;
	a.renorm = renorm;
	a.n_items = T * K * (EI / DEC_CHUNK);
	a.ncon = decode_ncon((size_t)T, (size_t)K, (size_t)EI, grid);
	a.off_start = (int)sl.off_start;
	a.off_rep = (int)sl.off_rep;
	a.rep_stride = (int)sl.rep_stride;
	a.spin = spin > 0 ? spin : MOE_SPIN_DEFAULT;
	a.norm_w = norm_w;
	a.x_out = x_out;
	void *args[] = {&a};
	hipError_t rc = hipLaunchKernel(norm_w ? g.fn_norm : g.fn, dim3(grid), dim3(g.NT), args,
					decode_lds_bytes(g, (size_t)E), (hipStream_t)stream);
	if (rc != hipSuccess)
		return (int)rc;
	return (int)hipGetLastError();
}

/* ---------------------------------------------------------------------- */
/* K-quant experts: routing and gate/up of a decode-sized call            */
/* ---------------------------------------------------------------------- */

/*
 * k_kq_route_gateup: the first of the two launches of a decode-sized layer
 * on K-quant experts (the second, k_kq_down_combine in kq_moe.hip, takes
 * the down products and the combine).  The reference's down product runs
 * one fp32 dot over all EI values of h per output (dot_f32_quant in
 * fused_ffn_silu, nn.c:483-492), so an output needs every h value of its
 * pair first: the launch boundary is that wait.
 *
 * Routing as k_moe_decode's (router rows by workgroups j < NE into tagged
 * replicas, softmax and top-k in every workgroup), with the same epoch,
 * start flags and poison rules.  Then units of R rows of the gate and R of
 * the up matrix of one (token, slot) pair p, R = NT / (2 * NB) so that a
 * unit is one super-block per thread: thread i takes super-block i % NB of
 * row i / NB (gate rows first, then up), its integer sums against the
 * token's Q8_K blocks (quantized by the workgroup while the routing is in
 * flight) go to LDS, and thread r < R runs row r's sequential steps
 * (dot_q4_K_q8_K / dot_q6_K_q8_K) for gate and up and writes h[p][row] =
 * (g / (1 + expf(-g))) * u (nn.c:455-478), bit for bit k_kq_gateup.  Each
 * workgroup takes a balanced contiguous range of the P * EI / R units; the
 * next unit's super-block is loaded while the current one's sums run.
 * Workgroup 0 writes the call's ids and weights.
 */
#define KQ_NT 512

template <int GT, int E, bool NORM>
__global__ __launch_bounds__(KQ_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_kq_route_gateup(DecodeArgs a)
{
	constexpr int NT = KQ_NT, NB = E / 256, R = NT / (2 * NB), RS = NB + 1;
	constexpr int QS = 65, BS = 17; /* token rows padded: distinct banks */
	constexpr int BY = kqb<GT>::BYTES, DW = GT == 3 ? 36 : 53;
	static_assert(2 * R * NB == NT, "a unit is one super-block per thread");
	extern __shared__ float lds[];
	__shared__ u32 s_ids[MOE_FUSED_MAX_P];
	__shared__ float s_w[MOE_FUSED_MAX_P];
	__shared__ u32 s_epoch;
	__shared__ u32 s_poison;
	__shared__ uint64_t s_tab[32];
	__shared__ int s_q8[NB * QS];
	__shared__ float s_d[NB];
	__shared__ int s_bs[NB * BS];
	__shared__ int s_rec[4][2 * R * RS];

	const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
	const int G = (int)gridDim.x, b = (int)blockIdx.x;
	const int CH = a.EI / R, N = a.n_items; /* units per pair, all units */
	const int u0 = item_lo(b, N, G), u1 = item_lo(b + 1, N, G);
	const size_t rb = (size_t)NB * BY;

	/* quantize_row_q8 of token t into s_q8 / s_bs / s_d (wave w takes
	 * blocks w, w + NT / 64, ...) */
	auto quantize = [&](int t) {
		for (int i = wave; i < NB; i += NT / WAVE) {
			const float4 v = ((const float4 *)(a.x + (size_t)t * E + (size_t)i * 256))[lane];
			float d;
			int bs;
			const u32 q = kg_q8k(v, lane, &d, &bs);
			s_q8[i * QS + lane] = (int)q;
			if (lane % 4 == 0)
				s_bs[i * BS + lane / 4] = bs;
			if (lane == 0)
				s_d[i] = d;
		}
	};
	/* this thread's super-block of unit u: matrix (gate, up), row, block */
	const int mat = tid / (R * NB), rl = (tid % (R * NB)) / NB, sb = tid % NB;
	auto load_unit = [&](int u, u32 (&w)[DW]) {
		const int p = u / CH, row = (u % CH) * R + rl;
		const uint8_t *blk = (mat ? a.up : a.gate) + (size_t)s_ids[p] * a.gu_stride +
				     (size_t)row * rb + (size_t)sb * BY;
		if constexpr (GT == 3)
			load_dwords<36>(blk, w);
		else
			kg_load<53>(blk, w);
	};

	if (tid < 32)
		s_tab[tid] = moe_exp2_tab[tid];
	u32 prev_epoch = 0, err0 = 0;
	if (tid == 0) { /* consumed late: the loads overlap routing */
		prev_epoch = ld_dev_u32(a.sync);
		err0 = ld_dev_u32(a.sync + MOE_SYNC_ERR_WORD);
	}
	if (b < a.NE)
		router_row<NT, E, NORM ? 2 : 0>(a, b, prev_epoch, lds, nullptr);
	/* the first unit's token does not depend on routing */
	int cur_t = -1;
	if (u0 < u1) {
		cur_t = u0 / CH / a.K;
		if constexpr (NORM) { /* one token, normalised here: wave w's
				       * block w + k NT / 64 is float4 tid + k NT */
			constexpr int NV = (E / 4 + NT - 1) / NT;
			float4 hv[NV];
			norm_token<NT, NV, 2>(a.x, a.norm_w, E, hv);
#pragma unroll
			for (int k = 0; k < NV; k++) {
				const int i = wave + k * (NT / WAVE);
				if (i < NB) {
					float d;
					int bs;
					const u32 q = kg_q8k(hv[k], lane, &d, &bs);
					s_q8[i * QS + lane] = (int)q;
					if (lane % 4 == 0)
						s_bs[i * BS + lane / 4] = bs;
					if (lane == 0)
						s_d[i] = d;
				}
			}
		} else {
			quantize(cur_t);
		}
	}
	if (tid == 0) {
		s_epoch = prev_epoch + 1;
		s_poison = err0;
	}
	__syncthreads();
	const u32 epoch = s_epoch;
	/* a wait of an earlier launch ran out (k_moe_decode's rule): NaN h,
	 * ids 0 and NaN weights, so the second launch writes NaN outputs; no
	 * start flag, no epoch advance */
	if (s_poison) {
		const float nan = __builtin_nanf("");
		for (int i = b * NT + tid; i < a.T * a.K * a.EI; i += G * NT)
			a.out[i] = nan;
		if (b == 0)
			for (int i = tid; i < a.T * a.K; i += NT) {
				a.ids_out[i] = 0;
				a.w_out[i] = nan;
			}
		return;
	}
	u32 *startf = a.sync + a.off_start;
	if (tid == 0 && b != 0)
		st_dev_u32(&startf[b], epoch);
	route_local<NT>(a, epoch, lds, s_ids, s_w, s_tab);
	if (b == 0)
		for (int i = tid; i < a.T * a.K; i += NT) {
			a.ids_out[i] = s_ids[i];
			a.w_out[i] = s_w[i];
		}

	u32 w[DW];
	if (u0 < u1)
		load_unit(u0, w);
	for (int u = u0; u < u1; u++) {
		const int p = u / CH, t = p / a.K;
		if (t != cur_t) { /* a later token: the previous unit's readers are done */
			quantize(t);
			cur_t = t;
		}
		__syncthreads(); /* the token's blocks; the previous unit's records read */
		float dsc, dmn = 0.0f;
		int sumi, msum = 0;
		if constexpr (GT == 3)
			kg_q4k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi, dmn, msum);
		else
			kg_q6k(w, s_q8 + sb * QS, s_bs + sb * BS, s_d[sb], dsc, sumi);
		if (u + 1 < u1) /* the next unit's block, in flight during the sums */
			load_unit(u + 1, w);
		const int slot = (mat * R + rl) * RS + sb;
		((float *)s_rec[0])[slot] = dsc;
		s_rec[1][slot] = sumi;
		((float *)s_rec[2])[slot] = dmn;
		s_rec[3][slot] = msum;
		__syncthreads();
		/* thread r < R: row r's steps for gate and up (dot_q4_K_q8_K
		 * returns acc + acc_m, dot_q6_K_q8_K acc) */
		if (tid < R) {
			float v[2];
#pragma unroll
			for (int m = 0; m < 2; m++) {
				const int o = (m * R + tid) * RS;
				float acc = 0.0f, acc_m = 0.0f;
#pragma unroll
				for (int i = 0; i < NB; i++) {
					acc = fmaf(((const float *)s_rec[0])[o + i], (float)s_rec[1][o + i],
						   acc);
					if constexpr (GT == 3)
						acc_m = fmaf(((const float *)s_rec[2])[o + i],
							     (float)s_rec[3][o + i], acc_m);
				}
				v[m] = GT == 3 ? acc + acc_m : acc;
			}
			const float g = v[0];
			a.out[(size_t)p * a.EI + (size_t)(u % CH) * R + tid] =
				(g / (1.0f + moe_expf(-g))) * v[1];
		}
	}

	/* workgroup 0 advances the epoch once every workgroup has read it (as
	 * k_moe_decode) */
	if (b != 0)
		return;
	if (wait_flags<NT>(startf + 1, G - 1, epoch, a.sync + MOE_SYNC_ERR_WORD, MOE_ERR_FLAGS,
			   a.spin) &&
	    tid == 0)
		st_dev_u32(a.sync, epoch);
}

static const void *kq_decode_fn(int gt, size_t E, bool norm = false)
{
#define KQPICK(G_, E_)                                                        \
	if (gt == G_ && E == E_)                                             \
		return norm ? (const void *)k_kq_route_gateup<G_, E_, true>          \
			    : (const void *)k_kq_route_gateup<G_, E_, false>;
	KQPICK(3, 1024)
	KQPICK(3, 2048)
	KQPICK(3, 4096)
	KQPICK(5, 1024)
	KQPICK(5, 2048)
	KQPICK(5, 4096)
#undef KQPICK
	return NULL;
}

/* dynamic LDS: the routing scratch (router row and token transposed, or
 * the per-wave top-k scratch) */
static size_t kq_decode_lds_bytes(size_t E)
{
	size_t rt = (size_t)2 * 8 * (E / 8 + 4) + CHAIN_OVERRUN;
	size_t tk = (size_t)(KQ_NT / WAVE) * (MOE_MAX_NE + 2 * MOE_MAX_TOPK);
	return (rt > tk ? rt : tk) * sizeof(float);
}

/* a decode-sized call of T tokens on gate/up type gt: the instance exists,
 * NE fits one wave's lanes, the pairs fit the routing slots, the units
 * divide d_ff (R = 256 / (E / 256) rows) */
extern "C" int moe_kq_decode_supported(int gt, size_t E, size_t EI, size_t NE, size_t T,
				       size_t K)
{
	if (!kq_decode_fn(gt, E) || NE > WAVE || NE == 0 || T == 0 ||
	    T * K > MOE_FUSED_MAX_P)
		return 0;
	const size_t R = KQ_NT / (2 * (E / 256));
	return EI % R == 0 && EI >= R;
}

/* one workgroup per CU, all resident (the routing waits on the router
 * workgroups), or 0 */
extern "C" int moe_kq_decode_grid(int gt, size_t E, size_t NE)
{
	const void *fn = kq_decode_fn(gt, E), *fn_n = kq_decode_fn(gt, E, true);
	int dev = 0, ncu = 0, per = 0, per_n = 0;
	if (!fn || hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		return 0;
	if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, KQ_NT,
							 kq_decode_lds_bytes(E)) != hipSuccess ||
	    per < 1 ||
	    hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_n, fn_n, KQ_NT,
							 kq_decode_lds_bytes(E)) != hipSuccess ||
	    per_n < 1)
		return 0;
	return ncu >= (int)NE && ncu >= MOE_FUSED_MAX_P ? ncu : 0;
}

extern "C" int moe_launch_kq_route_gateup(int gt, const float *x, const float *router,
					  const float *bias, const uint8_t *gate, const uint8_t *up,
					  size_t gu_stride, uint32_t *ids, float *w, float *h,
					  uint32_t *sync, int T, int E, int EI, int NE, int K,
					  int renorm, int grid, int spin, const float *norm_w,
					  float *x_out, void *stream)
{
	const void *fn = kq_decode_fn(gt, (size_t)E, norm_w != NULL);
	if (!fn || grid < NE || grid < T || (norm_w && (T != 1 || !x_out)) ||
	    !moe_kq_decode_supported(gt, (size_t)E, (size_t)EI, (size_t)NE, (size_t)T, (size_t)K))
		return (int)hipErrorInvalidValue;
	SyncLayout sl = sync_layout((size_t)T, (size_t)NE, grid);
	DecodeArgs a = {};
	a.x = x;
	a.router = router;
	a.bias = bias;
	a.gate = gate;
	a.up = up;
	a.gu_stride = gu_stride;
	a.ids_out = ids;
	a.w_out = w;
	a.out = h;
	a.sync = sync;
	a.T = T;
	a.E = E;
	a.EI = EI;
	a.NE = NE;
	a.K = K;
	a.renorm = renorm;
	a.n_items = T * K * (EI / (KQ_NT / (2 * (E / 256))));
	a.norm_w = norm_w;
	a.x_out = x_out;
	a.off_start = (int)sl.off_start;
	a.off_rep = (int)sl.off_rep;
	a.rep_stride = (int)sl.rep_stride;
	a.spin = spin > 0 ? spin : MOE_SPIN_DEFAULT;
	void *args[] = {&a};
	hipError_t rc = hipLaunchKernel(fn, dim3(grid), dim3(KQ_NT), args, kq_decode_lds_bytes(E),
					(hipStream_t)stream);
	if (rc != hipSuccess)
		return (int)rc;
	return (int)hipGetLastError();
}

/* ---------------------------------------------------------------------- */
/* static scratch of the allocation-free decode entry point               */
/* ---------------------------------------------------------------------- */

/*
 * The sync words, tagged partials, ids and weights of
 * hip_moe_ffn_dev_noalloc live here instead of in memory the layer
 * allocates.  Each device holds its own copy, at its own address, from the
 * time the module loads until the process ends.  In host code `scratch`
 * names a host-side stand-in, not device memory: host code only ever uses
 * the address hipGetSymbolAddress returns for the current device, kept per
 * device in g_scratch.
 */
static __device__ __align__(256) uint8_t scratch[MOE_STATIC_SCRATCH_BYTES];

#define MOE_SCRATCH_DEVICES 64
static void *g_scratch[MOE_SCRATCH_DEVICES];
static pthread_mutex_t g_scratch_mu = PTHREAD_MUTEX_INITIALIZER;

/* Once per device, with `dev` current: look up this device's copy of the
 * array and clear it (the epoch, error word and flags start at zero). */
extern "C" int moe_static_scratch_setup(int dev)
{
	if (dev < 0 || dev >= MOE_SCRATCH_DEVICES)
		return (int)hipErrorInvalidDevice;
	int rc = 0;
	pthread_mutex_lock(&g_scratch_mu);
	if (!g_scratch[dev]) {
		void *p = NULL;
		hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
		if (e == hipSuccess && p)
			e = hipMemset(p, 0, MOE_STATIC_SCRATCH_BYTES);
		if (e == hipSuccess)
			e = hipDeviceSynchronize();
		if (e == hipSuccess)
			g_scratch[dev] = p;
		rc = (int)e;
	}
	pthread_mutex_unlock(&g_scratch_mu);
	return rc;
}

/* This device's copy of the array, NULL before moe_static_scratch_setup. */
extern "C" void *moe_static_scratch(int dev)
{
	if (dev < 0 || dev >= MOE_SCRATCH_DEVICES)
		return NULL;
	pthread_mutex_lock(&g_scratch_mu);
	void *p = g_scratch[dev];
	pthread_mutex_unlock(&g_scratch_mu);
	return p;
}

#ifdef MOE_STAGE_STAMPS
/* the stage stamps of the last launch: [MOE_STAMP_WGS][MOE_STAMPS] */
extern "C" int moe_stage_stamps(unsigned long long *out)
{
	return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_stage_stamps), sizeof(g_stage_stamps), 0,
					 hipMemcpyDeviceToHost);
}
#endif
