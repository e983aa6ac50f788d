/*
 * moe_qgemv.hip - dense quantized matrix product for gfx950:
 *   out[t][j] = add[t][j] (or add[j]) + dot(x[t], W[j])      (add optional)
 * with W a row-major matrix of N rows of K columns in Q8_0 or Q4_0 blocks.
 *
 * This is the reference's tensor_mma_transposed_2x2 with a quantized right
 * operand (matmul.c:451-462 -> 270-324: result = add or 0, then
 * result[t][j] += dot, matmul.c:13-33), which its models call for the
 * attention projections (olmoe.c:448-450), the output projection and the
 * lm_head (olmoe.c:563,577), and its fused_gemv2/3 (nn.c:340-425: the same
 * dots over consecutive weight segments).  The reference's default build
 * (-DQ8_DOT, Makefile:29) takes dot_q8_quant per element for any T
 * (matmul.c:107-131,145-165,285-312), which for Q8_0/Q4_0 is dot_f32_quant
 * (quant.c:577-614,656-668).  The dots here are the same products in
 * another order (two blocks per lane, then a lane tree), and each block's
 * sum is taken as d * (sum((q + c) x) - c * sum(x)) with c = 128 (Q8_0) or
 * 8 (Q4_0), the biased quant bytes converted directly.  Error bound, first
 * order, per output: 2^-24 * (32 (127 + c) + 31 c + 64 * 255) * B with
 * B = sum over blocks of |d| * sum |x| (the offset's cancellation makes it
 * grow with sum |x|, not with |sum q x|).  Measured: ~1e-6 relative L2 on
 * zero-mean activations, 1e-5 or less with a mean 16 times the spread.
 *
 * Bound: HBM.  Algorithmic bytes per call: N * K/32 * block bytes (34 for
 * Q8_0, 18 for Q4_0) + T*K*4 (x) + T*N*4 (out) (+ T*N*4 with add).
 *
 * Geometry: C = K/64 lanes per row (a power of two, 4..64), each lane one
 * 64-column segment (two blocks) of a row; a row group is 64/C rows per
 * wave, four waves.  As many workgroups as the chip holds at once (the
 * occupancy of the instance times the CUs, moe_qgemv_grid) walk the row
 * groups (g, g + grid, ...), loading the next group's segments while the
 * current one's dots run.  Measured with fixed grids of 512 / 768 / 1024 /
 * 2048: OLMoE lm_head (Q8_0, 3 workgroups per CU) 24.5 / 22.0 / 27.1 /
 * 24.8 us, Mixtral lm_head (Q4_0, 5 per CU) 23.5 / 20.5 / 19.8 / 20.8 us:
 * a grid past what is resident leaves a second partial round.  The tokens
 * are staged in LDS tg at a time (up to 4, within QG_LDS_MAX; each segment
 * padded by 4 floats so the C lanes of a row read distinct banks): once per
 * workgroup when they all fit (one token: see k_qgemv1), every token reusing
 * the registers' weights, so W is read from HBM once.  With more tokens
 * than that, the token groups go outside and the workgroup's row groups
 * inside: each group of tokens is staged once and the weights load again
 * per group, mostly from L2 (sixteen tokens of 4096 columns: 6 groups of 3).
 * (One pass of a
 * workgroup per row group measured 26.3 us for the OLMoE lm_head and 32.2
 * for Mixtral's: every workgroup staged the token again, 51 and 128 MB of
 * L2 reads.)
 */
#include "moe_qgemv.h"

static size_t qg_tok_bytes(int K)
{
	return (size_t)(K / MOE_SEG_COLS) * SEG_STRIDE * sizeof(float);
}

static int qg_tgmax(int K, int T)
{
	return min(T, min(4, (int)(QG_LDS_MAX / qg_tok_bytes(K))));
}

/* one token: its columns stay in LDS (read at each use), which with a
 * request for 4 waves per SIMD keeps the Q8_0 instance at ~111 VGPRs
 * without spills (3 waves per SIMD at 138 VGPRs with the columns held in
 * registers: 22.1 us against 20.8 for the OLMoE lm_head); the Q4_0
 * instance stays at 5 waves either way */
template <int WT, int C>
__global__ __launch_bounds__(QG_WAVES * WAVE)
__attribute__((amdgpu_waves_per_eu(4))) void k_qgemv1(QG_ARGS)
{
	extern __shared__ __attribute__((aligned(16))) float sx1[];
	qgemv_body<WT, C, true>(sx1, W, rb, N, K, x, T, tgmax, add, add_rows, out);
}

/* several tokens (requesting 4 waves per SIMD here spills the Q8_0 instance) */
template <int WT, int C>
__global__ __launch_bounds__(QG_WAVES * WAVE) void k_qgemv(QG_ARGS)
{
	extern __shared__ __attribute__((aligned(16))) float sxn[];
	qgemv_body<WT, C, false>(sxn, W, rb, N, K, x, T, tgmax, add, add_rows, out);
}

template <int WT>
static int launch_qgemv_t(int C, const uint8_t *W, size_t rb, int N, int K, const float *x,
			  int T, const float *add, int add_rows, float *out, int nwg,
			  hipStream_t s)
{
	const int ngroups = (N + QG_WAVES * (WAVE / C) - 1) / (QG_WAVES * (WAVE / C));
	const dim3 grid(min(ngroups, nwg > 0 ? nwg : QG_GRID));
	const int tgmax = qg_tgmax(K, T);
	const size_t lds = (size_t)tgmax * qg_tok_bytes(K);
#define QG(CC)                                                                          \
	case CC:                                                                        \
		if (T == 1)                                                             \
			hipLaunchKernelGGL((k_qgemv1<WT, CC>), grid, dim3(QG_WAVES * WAVE),      \
					   lds, s, W, rb, N, K, x, T, tgmax, add, add_rows, \
					   out);                                        \
		else                                                                    \
			hipLaunchKernelGGL((k_qgemv<WT, CC>), grid,                      \
					   dim3(QG_WAVES * WAVE), lds, s, W, rb, N, K, x, T, \
					   tgmax, add, add_rows, out);                  \
		break;
	switch (C) {
		QG(4) QG(8) QG(16) QG(32) QG(64)
	default:
		return (int)hipErrorInvalidValue;
	}
#undef QG
	return (int)hipGetLastError();
}

/* resident workgroups of the instance for (wtype, K, T == 1 or not) times
 * the CUs of the current device; 0 if the query fails */
extern "C" int moe_qgemv_grid(int wtype, int K, int one)
{
	const int C = moe_lanes_per_row((size_t)K);
	const size_t lds = (size_t)qg_tgmax(K, one ? 1 : 4) * qg_tok_bytes(K);
	int dev = 0, ncu = 0, per = 0;
	hipError_t e = hipSuccess;
	if (hipGetDevice(&dev) != hipSuccess ||
	    hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
		return 0;
#define OCC(WTT, CC)                                                                        \
	if (wtype == WTT && C == CC)                                                        \
		e = one ? hipOccupancyMaxActiveBlocksPerMultiprocessor(                      \
				  &per, k_qgemv1<WTT, CC>, QG_WAVES * WAVE, lds)           \
			: hipOccupancyMaxActiveBlocksPerMultiprocessor(                      \
				  &per, k_qgemv<WTT, CC>, QG_WAVES * WAVE, lds);
	OCC(1, 4) OCC(1, 8) OCC(1, 16) OCC(1, 32) OCC(1, 64)
	OCC(2, 4) OCC(2, 8) OCC(2, 16) OCC(2, 32) OCC(2, 64)
#undef OCC
	if (e != hipSuccess || per < 1)
		return 0;
	return per * ncu;
}

extern "C" int moe_launch_qgemv(int wtype, const uint8_t *W, int N, int K, const float *x,
				int T, const float *add, int add_rows, float *out, int nwg,
				void *stream)
{
	const int C = moe_lanes_per_row((size_t)K);
	if (N < 1 || T < 1 || K < 256 || K % 256 || moe_kchunks((size_t)K) != 1 || C < 4)
		return (int)hipErrorInvalidValue;
	const size_t rb = (size_t)(K / MOE_QK) * (wtype == 1 ? 34 : 18);
	hipStream_t s = (hipStream_t)stream;
	if (wtype == 1)
		return launch_qgemv_t<1>(C, W, rb, N, K, x, T, add, add_rows, out, nwg, s);
	if (wtype == 2)
		return launch_qgemv_t<2>(C, W, rb, N, K, x, T, add, add_rows, out, nwg, s);
	return (int)hipErrorInvalidValue;
}
