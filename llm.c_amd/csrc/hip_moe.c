/*
 * hip_moe.c - thin C host layer of the MI355X MoE FFN (see include/hip_moe.h).
 *
 * Owns device residency of one layer's weights (uploaded once as GGUF
 * blocks: gate/up rows unchanged, down matrices regrouped by whole blocks
 * into panels, see upload_down), per-layer scratch, and the launch sequence
 *   router -> softmax/top-k -> gate/up + SwiGLU -> down -> combine
 * that replaces the per-token loop of moe_ffn (olmoe.c:359-406,
 * llama.c:409-456).  Errors follow the reference's "return 0, caller falls
 * back" convention of fused_ffn_silu (nn.c:496-539): nothing here aborts.
 */
#include "hip_moe.h"
#include "moe_internal.h"

#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct hip_moe_layer {
	int wtype;          /* the gate/up block type */
	int dtype;          /* the down block type */
	int kq;             /* K-quant experts: the kq_moe.hip path */
	size_t E, EI, NE, topk;
	int renorm;
	int device;

	size_t rb_in;       /* bytes of one row with E columns */
	size_t rb_mid;      /* bytes of one row with EI columns */
	size_t gu_stride;   /* bytes of one expert's gate (or up) matrix */
	size_t down_stride; /* bytes of one expert's down matrix */

	float *d_router;
	uint8_t *d_weights; /* [gate NE][up NE][down NE] ([gate NE][up NE] grouped) */
	uint8_t *d_gate, *d_up, *d_down;
	uint8_t *d_gate_g, *d_up_g; /* gate/up in MOE_GU_GROUP-row groups (grouped path) */
	size_t weight_bytes;

	hipStream_t stream;
	int fused_grid;     /* workgroups of the persistent kernel, 0 = none */
	int path;           /* HIP_MOE_PATH_*, AUTO unless set */
	int spin;           /* poll rounds of a decode-kernel wait, 0 = MOE_SPIN_DEFAULT */

	/* scratch for up to cap_T tokens; scratch_gen counts its reallocations
	 * (a graph captured before one names freed buffers) */
	size_t cap_T;
	unsigned scratch_gen;
	int used_static;    /* a hip_moe_ffn_dev_noalloc call ran on this layer */
	float *d_logits;
	uint32_t *d_ids;
	float *d_w;
	float *d_h;
	float *d_ypart;     /* fp32 partials of the GEMV and grouped paths */
	size_t ypart_cap;   /* floats */
	uint64_t *d_part;   /* epoch-tagged partials of the decode kernel */
	size_t part_words;
	uint32_t *d_sync;   /* epoch and flags of the decode kernel */
	size_t sync_words;
	int *d_rows;        /* grouped path: sorted pair per row, -1 = padding */
	int *d_tile_e;      /* grouped path: expert of each m-tile, -1 = unused */
	void *d_h16;        /* grouped path: f16 h in sorted row order */
	void *d_xh;         /* grouped path: tokens rounded to f16 [T][E] */

	/* staging for the host-pointer entry point */
	size_t cap_io;
	float *d_x, *d_out, *d_bias;
	uint32_t *d_ids_io;
	float *d_w_io;
};

static __thread char g_err[512];

static void set_err(const char *fmt, ...)
{
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(g_err, sizeof(g_err), fmt, ap);
	va_end(ap);
	fprintf(stderr, "hip_moe: %s\n", g_err);
}

const char *hip_moe_last_error(void)
{
	return g_err;
}

void moe_set_error(const char *msg)
{
	set_err("%s", msg);
}

#define HIPCHK(call, what)                                                        \
	do {                                                                      \
		hipError_t e_ = (call);                                           \
		if (e_ != hipSuccess) {                                           \
			set_err("%s: %s", what, hipGetErrorString(e_));            \
			goto fail;                                                \
		}                                                                 \
	} while (0)

#define LCHK(rc, what)                                                            \
	do {                                                                      \
		int r_ = (rc);                                                    \
		if (r_ != 0) {                                                    \
			set_err("%s: %s", what, hipGetErrorString((hipError_t)r_)); \
			return 0;                                                 \
		}                                                                 \
	} while (0)

/*
 * One library stream per device, shared by every layer: calls that pass no
 * stream run in call order, as the reference's layers do.  A decode launch
 * keeps one workgroup on every CU and its workgroups wait on one another, so
 * two decode launches in flight at once (two streams) can each hold CUs the
 * other needs; they then end on their bounded waits with an error instead of
 * finishing.  One stream rules that out for the default.
 */
#define MOE_MAX_DEVICES 64
static hipStream_t g_dev_stream[MOE_MAX_DEVICES];
static pthread_mutex_t g_dev_stream_mu = PTHREAD_MUTEX_INITIALIZER;

static hipStream_t device_stream(int dev)
{
	hipStream_t s = NULL;
	if (dev < 0 || dev >= MOE_MAX_DEVICES) {
		set_err("device %d: beyond the %d devices this library serves", dev,
			MOE_MAX_DEVICES);
		return NULL;
	}
	pthread_mutex_lock(&g_dev_stream_mu);
	if (!g_dev_stream[dev]) {
		hipError_t e = hipStreamCreateWithFlags(&g_dev_stream[dev], hipStreamNonBlocking);
		if (e != hipSuccess) {
			g_dev_stream[dev] = NULL;
			set_err("hipStreamCreate: %s", hipGetErrorString(e));
		}
	}
	s = g_dev_stream[dev];
	pthread_mutex_unlock(&g_dev_stream_mu);
	return s;
}

static size_t row_bytes(int wtype, size_t n)
{
	if (wtype == HIP_MOE_Q4_K || wtype == HIP_MOE_Q6_K)
		return (n / 256) * (wtype == HIP_MOE_Q4_K ? 144 : 210);
	return (n / MOE_QK) * (wtype == HIP_MOE_Q8_0 ? 34 : 18);
}

static int is_kquant(int wtype)
{
	return wtype == HIP_MOE_Q4_K || wtype == HIP_MOE_Q6_K;
}

static int is_pow2(size_t v)
{
	return v && !(v & (v - 1));
}

/*
 * Expert e's down matrix [E rows][EI/32 blocks] (GGUF order) goes to the
 * device as EI/32 panels: panel c = block c of rows 0..E-1, contiguous.
 * Only whole blocks move, so every block keeps its bytes; a decode item
 * (32 columns of down for all E rows) then reads one contiguous panel, and
 * the down GEMV and GEMM read E-row runs of blocks.
 */
/*
 * One expert's gate or up matrix [EI][E] (GGML rows) into MOE_GU_GROUP-row
 * groups, piece-major inside a group: piece s (blocks 2s, 2s+1) of row r
 * goes to (r / G) * G * rb + s * G * pb + (r % G) * pb.  Blocks keep their
 * bytes; only their order changes.
 */
static int upload_gu(hip_moe_layer *L, uint8_t *dst, const uint8_t *src, uint8_t *stage)
{
	const size_t G = MOE_GU_GROUP, rb = L->rb_in, pb = 2 * (rb / (L->E / MOE_QK));
	const size_t np = L->E / (2 * MOE_QK);
	for (size_t r = 0; r < L->EI; r++)
		for (size_t s = 0; s < np; s++)
			memcpy(stage + (r / G) * G * rb + s * G * pb + (r % G) * pb,
			       src + r * rb + s * pb, pb);
	HIPCHK(hipMemcpy(dst, stage, L->gu_stride, hipMemcpyHostToDevice), "upload gate/up");
	return 1;
fail:
	return 0;
}

static int upload_down(hip_moe_layer *L, size_t e, const uint8_t *src, uint8_t *stage)
{
	const size_t bb = L->wtype == HIP_MOE_Q8_0 ? 34 : 18, nc = L->EI / MOE_QK;
	for (size_t i = 0; i < L->E; i++) {
		const uint8_t *row = src + i * L->rb_mid;
		for (size_t c = 0; c < nc; c++)
			memcpy(stage + (c * L->E + i) * bb, row + c * bb, bb);
	}
	HIPCHK(hipMemcpy(L->d_down + e * L->down_stride, stage, L->down_stride,
			 hipMemcpyHostToDevice), "upload down");
	return 1;
fail:
	return 0;
}

void hip_moe_free(hip_moe_layer *L)
{
	if (!L)
		return;
	hipFree(L->d_router);
	hipFree(L->d_weights);
	hipFree(L->d_logits);
	hipFree(L->d_ids);
	hipFree(L->d_w);
	hipFree(L->d_h);
	hipFree(L->d_ypart);
	hipFree(L->d_part);
	hipFree(L->d_sync);
	hipFree(L->d_rows);
	hipFree(L->d_tile_e);
	hipFree(L->d_h16);
	hipFree(L->d_xh);
	hipFree(L->d_x);
	hipFree(L->d_out);
	hipFree(L->d_bias);
	hipFree(L->d_ids_io);
	hipFree(L->d_w_io);
	free(L); /* L->stream is the device's shared stream: it stays */
}

hip_moe_layer *hip_moe_upload(const float *gate_inp, const void *const *gate_e,
			      const void *const *up_e, const void *const *down_e,
			      int wtype, size_t E, size_t EI, size_t NE, size_t topk,
			      int renorm)
{
	return hip_moe_upload_typed(gate_inp, gate_e, up_e, down_e, wtype, wtype, E, EI, NE,
				    topk, renorm);
}

hip_moe_layer *hip_moe_upload_typed(const float *gate_inp, const void *const *gate_e,
				    const void *const *up_e, const void *const *down_e,
				    int gate_type, int down_type, size_t E, size_t EI, size_t NE,
				    size_t topk, int renorm)
{
	hip_moe_layer *L = NULL;
	uint8_t *stage = NULL;
	int ndev = 0;
	const int wtype = gate_type;
	const int kq = is_kquant(gate_type) && is_kquant(down_type);

	if (!kq && (gate_type != down_type ||
		    (gate_type != HIP_MOE_Q8_0 && gate_type != HIP_MOE_Q4_0))) {
		set_err("upload: unsupported weight types %d/%d (Q8_0=1 or Q4_0=2 for all three "
			"matrices; Q4_K=3 / Q6_K=5 for gate/up and down in any mix)", gate_type,
			down_type);
		return NULL;
	}
	if (!gate_inp || !gate_e || !up_e || !down_e) {
		set_err("upload: NULL weight pointer");
		return NULL;
	}
	if (E == 0 || EI == 0 || E % 256 || EI % 256) {
		set_err("upload: E=%zu and EI=%zu must be non-zero multiples of 256", E, EI);
		return NULL;
	}
	/* gate/up rows are covered by one wave without K-split: E/64 lanes */
	if (!kq && (!is_pow2(E / MOE_SEG_COLS) || E / MOE_SEG_COLS > 64)) {
		set_err("upload: E=%zu not supported (needs E/64 a power of two <= 64)", E);
		return NULL;
	}
	if (kq && !moe_kq_layer_supported(gate_type, down_type, E, EI)) {
		set_err("upload: E=%zu EI=%zu not supported for K-quant experts (E <= 8192, "
			"EI <= 16384)", E, EI);
		return NULL;
	}
	if (NE == 0 || NE > MOE_MAX_NE || topk == 0 || topk > NE || topk > MOE_MAX_TOPK) {
		set_err("upload: NE=%zu topk=%zu out of range (1<=topk<=NE<=%d, topk<=%d)",
			NE, topk, MOE_MAX_NE, MOE_MAX_TOPK);
		return NULL;
	}
	if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
		set_err("upload: no HIP device");
		return NULL;
	}

	L = calloc(1, sizeof(*L));
	if (!L) {
		set_err("upload: out of host memory");
		return NULL;
	}
	L->wtype = wtype;
	L->dtype = down_type;
	L->kq = kq;
	L->E = E;
	L->EI = EI;
	L->NE = NE;
	L->topk = topk;
	L->renorm = renorm ? 1 : 0;
	L->rb_in = row_bytes(wtype, E);
	L->rb_mid = row_bytes(down_type, EI);
	L->gu_stride = EI * L->rb_in;
	L->down_stride = E * L->rb_mid;
	/* the grouped GEMMs read gate/up from a second copy in MOE_GU_GROUP-row
	 * groups (a K-step is one contiguous run per group); the decode and GEMV
	 * kernels read whole rows from the first.  K-quant experts stay as
	 * they are (rows of super-blocks), for the kq_moe.hip kernels only. */
	const int grouped = !kq && moe_prefill_supported(wtype, E, EI, NE);
	const size_t wbytes = NE * (2 * L->gu_stride + L->down_stride) +
			      (grouped ? 2 * NE * L->gu_stride : 0);
	L->weight_bytes = NE * E * sizeof(float) + wbytes;
	/* the persistent first launch of the decode path (K-quants: routing
	 * and gate/up) */
	L->fused_grid = kq ? moe_kq_decode_grid(wtype, E, NE) : moe_fused_grid(wtype, E, EI, NE);

	HIPCHK(hipGetDevice(&L->device), "hipGetDevice");
	L->stream = device_stream(L->device);
	if (!L->stream)
		goto fail;
	/* once per device: the static scratch of hip_moe_ffn_dev_noalloc */
	HIPCHK((hipError_t)moe_static_scratch_setup(L->device), "static scratch set-up");
	HIPCHK(hipMalloc((void **)&L->d_router, NE * E * sizeof(float)), "hipMalloc(router)");
	/* + slack: readable bytes past the last weight */
	HIPCHK(hipMalloc((void **)&L->d_weights, wbytes + MOE_WEIGHT_SLACK), "hipMalloc(experts)");
	L->d_gate = L->d_weights;
	L->d_up = L->d_gate + NE * L->gu_stride;
	L->d_down = L->d_up + NE * L->gu_stride;
	if (grouped) {
		L->d_gate_g = L->d_down + NE * L->down_stride;
		L->d_up_g = L->d_gate_g + NE * L->gu_stride;
	}
	HIPCHK(hipMemset(L->d_weights + wbytes, 0, MOE_WEIGHT_SLACK), "clear slack");

	HIPCHK(hipMemcpy(L->d_router, gate_inp, NE * E * sizeof(float), hipMemcpyHostToDevice),
	       "upload router");
	stage = malloc(L->down_stride);
	if (!stage) {
		set_err("upload: out of host memory");
		goto fail;
	}
	for (size_t e = 0; e < NE; e++) {
		if (!gate_e[e] || !up_e[e] || !down_e[e]) {
			set_err("upload: NULL pointer for expert %zu", e);
			goto fail;
		}
		HIPCHK(hipMemcpy(L->d_gate + e * L->gu_stride, gate_e[e], L->gu_stride,
				 hipMemcpyHostToDevice), "upload gate");
		HIPCHK(hipMemcpy(L->d_up + e * L->gu_stride, up_e[e], L->gu_stride,
				 hipMemcpyHostToDevice), "upload up");
		if (kq)
			HIPCHK(hipMemcpy(L->d_down + e * L->down_stride, down_e[e], L->down_stride,
					 hipMemcpyHostToDevice), "upload down");
		else if (!upload_down(L, e, (const uint8_t *)down_e[e], stage))
			goto fail;
		if (grouped &&
		    (!upload_gu(L, L->d_gate_g + e * L->gu_stride, (const uint8_t *)gate_e[e], stage) ||
		     !upload_gu(L, L->d_up_g + e * L->gu_stride, (const uint8_t *)up_e[e], stage)))
			goto fail;
	}
	free(stage);
	return L;
fail:
	free(stage);
	hip_moe_free(L);
	return NULL;
}

size_t hip_moe_weight_bytes(const hip_moe_layer *L)
{
	return L ? L->weight_bytes : 0;
}

/*
 * Scratch for calls of up to T tokens.  Growing it frees the old buffers,
 * which a HIP graph captured earlier would still name, so growth is refused
 * while `s` is capturing: reserve first (hip_moe_reserve).
 */
static int ensure_scratch(hip_moe_layer *L, size_t T, hipStream_t s)
{
	if (T <= L->cap_T)
		return 1;
	size_t P = T * L->topk;
	hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
	HIPCHK(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing");
	if (cs != hipStreamCaptureStatusNone) {
		set_err("scratch holds %zu tokens, the call has %zu: growing it under stream "
			"capture would free buffers a graph names (reserve with hip_moe_reserve "
			"before capturing)", L->cap_T, T);
		return 0;
	}
	/* calls enqueued earlier may still use the buffers freed here */
	HIPCHK(hipDeviceSynchronize(), "synchronize before growing scratch");
	hipFree(L->d_logits);
	hipFree(L->d_ids);
	hipFree(L->d_w);
	hipFree(L->d_h);
	hipFree(L->d_ypart);
	hipFree(L->d_part);
	hipFree(L->d_sync);
	hipFree(L->d_rows);
	hipFree(L->d_tile_e);
	hipFree(L->d_h16);
	hipFree(L->d_xh);
	L->d_part = NULL;
	L->d_xh = NULL;
	L->d_rows = NULL;
	L->d_tile_e = NULL;
	L->d_h16 = NULL;
	L->d_logits = NULL;
	L->d_ids = NULL;
	L->d_w = NULL;
	L->d_h = NULL;
	L->d_ypart = NULL;
	L->d_sync = NULL;
	L->cap_T = 0;
	HIPCHK(hipMalloc((void **)&L->d_logits, T * L->NE * sizeof(float)), "hipMalloc(logits)");
	HIPCHK(hipMalloc((void **)&L->d_ids, P * sizeof(uint32_t)), "hipMalloc(ids)");
	HIPCHK(hipMalloc((void **)&L->d_w, P * sizeof(float)), "hipMalloc(w)");
	HIPCHK(hipMalloc((void **)&L->d_h, P * L->EI * sizeof(float)), "hipMalloc(h)");
	/* fp32 partials of the GEMV (its K-chunks) and grouped paths (their
	 * K-splits: room for several when the pairs are few) */
	L->ypart_cap = moe_down_part_floats(L->E, L->EI, P);
	if (L->ypart_cap < P * L->E * 2)
		L->ypart_cap = P * L->E * 2;
	if (L->ypart_cap < ((size_t)1 << 22))
		L->ypart_cap = (size_t)1 << 22;
	HIPCHK(hipMalloc((void **)&L->d_ypart, L->ypart_cap * sizeof(float)), "hipMalloc(ypart)");
	/* decode kernel: epoch-tagged partials, for every T it can take up to
	 * this capacity */
	L->part_words = 1;
	for (size_t t = 1; !L->kq && L->fused_grid > 0 && t <= T && t * L->topk <= MOE_FUSED_MAX_P;
	     t++) {
		size_t w = moe_fused_part_words(t, L->topk, L->E, L->EI, L->fused_grid);
		L->part_words = w > L->part_words ? w : L->part_words;
	}
	HIPCHK(hipMalloc((void **)&L->d_part, L->part_words * sizeof(uint64_t)), "hipMalloc(part)");
	L->sync_words = moe_fused_sync_words(T, L->NE, L->fused_grid > 0 ? L->fused_grid : 1);
	HIPCHK(hipMalloc((void **)&L->d_sync, L->sync_words * sizeof(uint32_t)), "hipMalloc(sync)");
	/* zeroed once here: the decode kernel's flags and its partials carry an
	 * epoch that starts at 1, and reused device memory may hold tags of an
	 * earlier layer */
	HIPCHK(hipMemset(L->d_sync, 0, L->sync_words * sizeof(uint32_t)), "hipMemset(sync)");
	HIPCHK(hipMemset(L->d_part, 0, L->part_words * sizeof(uint64_t)), "hipMemset(part)");
	/* the clears run on the null stream, which the layer's non-blocking
	 * stream does not wait for */
	HIPCHK(hipDeviceSynchronize(), "synchronize after clearing scratch");
	if (!L->kq && moe_prefill_supported(L->wtype, L->E, L->EI, L->NE)) {
		size_t rows = moe_prefill_max_rows(P, L->NE);
		HIPCHK(hipMalloc((void **)&L->d_rows, rows * sizeof(int)), "hipMalloc(rows)");
		HIPCHK(hipMalloc((void **)&L->d_tile_e,
				 moe_prefill_tile_ints(P, L->NE) * sizeof(int)),
		       "hipMalloc(tiles)");
		HIPCHK(hipMalloc(&L->d_h16, rows * L->EI * 2), "hipMalloc(h16)");
		HIPCHK(hipMalloc(&L->d_xh, T * L->E * 2), "hipMalloc(xh)");
	}
	L->cap_T = T;
	L->scratch_gen++;
	return 1;
fail:
	return 0;
}

unsigned moe_scratch_gen(const hip_moe_layer *L)
{
	return L ? L->scratch_gen : 0;
}

static int check_T(size_t T);

static hipStream_t pick_stream(hip_moe_layer *L, void *stream)
{
	return stream ? (hipStream_t)stream : L->stream;
}

int hip_moe_reserve(hip_moe_layer *L, size_t T)
{
	if (!L) {
		set_err("reserve: NULL layer");
		return 0;
	}
	if (T == 0 || T > 65535) {
		set_err("reserve: token count %zu out of range 1..65535", T);
		return 0;
	}
	return ensure_scratch(L, T, L->stream);
}

int hip_moe_set_wait_limit(hip_moe_layer *L, int polls)
{
	if (!L || polls < 0) {
		set_err("set_wait_limit: bad layer or poll count %d", polls);
		return 0;
	}
	L->spin = polls;
	return 1;
}

/*
 * Read the decode kernel's error word after `s` drains; if a wait ran out,
 * clear the sync words and partials (the device is idle then) so that the
 * epoch restarts, and report the code.  0 = no error, > 0 = MOE_ERR_*,
 * -1 = the query itself failed.
 */
static int check_and_reset(hip_moe_layer *L, hipStream_t s)
{
	uint32_t err = 0;
	HIPCHK(hipStreamSynchronize(s), "synchronize");
	if (!L->d_sync)
		return 0;
	HIPCHK(hipMemcpy(&err, L->d_sync + MOE_SYNC_ERR_WORD, sizeof(err), hipMemcpyDeviceToHost),
	       "read error word");
	if (!err)
		return 0;
	/* every launch since the failed one returned NaN outputs; flags may be
	 * left mid-flight: restart the epoch at zero */
	HIPCHK(hipDeviceSynchronize(), "synchronize before reset");
	HIPCHK(hipMemset(L->d_sync, 0, L->sync_words * sizeof(uint32_t)), "clear sync words");
	HIPCHK(hipMemset(L->d_part, 0, L->part_words * sizeof(uint64_t)), "clear partials");
	HIPCHK(hipDeviceSynchronize(), "synchronize after reset");
	static const char *what[] = {"", "router logits", "partial sums", "start flags"};
	set_err("persistent kernel: a dependency wait timed out (%s); outputs of that call "
		"and of the calls after it until this report are invalid (NaN)",
		err < 4 ? what[err] : "unknown");
	return (int)err;
fail:
	return -1;
}

/* the same check for the device's static scratch (hip_moe_ffn_dev_noalloc) */
static int check_and_reset_static(int dev)
{
	uint8_t *base = (uint8_t *)moe_static_scratch(dev);
	uint32_t err = 0;
	if (!base)
		return 0;
	HIPCHK(hipMemcpy(&err, base + MOE_SYNC_ERR_WORD * sizeof(uint32_t), sizeof(err),
			 hipMemcpyDeviceToHost), "read static error word");
	if (!err)
		return 0;
	HIPCHK(hipDeviceSynchronize(), "synchronize before reset");
	HIPCHK(hipMemset(base, 0, MOE_STATIC_SCRATCH_BYTES), "clear static scratch");
	HIPCHK(hipDeviceSynchronize(), "synchronize after reset");
	set_err("persistent kernel (static scratch): a dependency wait timed out (code %u); "
		"outputs of hip_moe_ffn_dev_noalloc since then are invalid (NaN)", err);
	return (int)err;
fail:
	return -1;
}

int hip_moe_status(hip_moe_layer *L, void *stream)
{
	if (!L) {
		set_err("status: NULL layer");
		return -1;
	}
	int rc = check_and_reset(L, pick_stream(L, stream));
	/* the device's static scratch only for a layer that ran there: another
	 * caller of the no-allocation entry point may still be using it */
	int rs = rc < 0 || !L->used_static ? 0 : check_and_reset_static(L->device);
	return rc != 0 ? rc : rs;
}

/*
 * The decode path of hip_moe_ffn_dev with its scratch (sync words, tagged
 * partials, ids and weights when the caller passes none) in the device's
 * static array instead of the layer's buffers: no allocation, no memset,
 * no synchronisation.  Layout in the array: sync words at 0, partials from
 * the sync size of the layer's largest decode call (256-byte aligned), then
 * ids and weights.  Every call on a device shares that array; the epoch
 * tags make the contents a previous call left (of any size or layer) stale.
 */
int hip_moe_ffn_dev_noalloc(hip_moe_layer *L, const float *d_x, float *d_out, size_t T,
			    const float *d_router_bias, uint32_t *d_ids_out, float *d_w_out,
			    void *stream)
{
	if (!L || !d_x || !d_out) {
		set_err("ffn_noalloc: NULL argument");
		return 0;
	}
	if (!check_T(T))
		return 0;
	if (L->kq) {
		set_err("ffn_noalloc: K-quant experts take the layer's own scratch "
			"(hip_moe_ffn_dev)");
		return 0;
	}
	if (L->fused_grid <= 0 ||
	    !moe_fused_supported(L->wtype, L->E, L->EI, L->NE, T, L->topk) ||
	    (L->path != HIP_MOE_PATH_AUTO && L->path != HIP_MOE_PATH_DECODE)) {
		set_err("ffn_noalloc: only the decode path (T*topk <= %d) runs without "
			"allocation; T=%zu topk=%zu does not take it", MOE_FUSED_MAX_P, T, L->topk);
		return 0;
	}
	uint8_t *base = (uint8_t *)moe_static_scratch(L->device);
	if (!base) {
		set_err("ffn_noalloc: the static scratch of device %d is not set up", L->device);
		return 0;
	}
	const size_t tmax = MOE_FUSED_MAX_P / L->topk;
	const size_t part_off =
		(moe_fused_sync_words(tmax, L->NE, L->fused_grid) * sizeof(uint32_t) + 255) &
		~(size_t)255;
	const size_t part_bytes =
		moe_fused_part_words(T, L->topk, L->E, L->EI, L->fused_grid) * sizeof(uint64_t);
	const size_t ids_off = part_off + part_bytes, P = T * L->topk;
	const size_t need = ids_off + 2 * P * sizeof(uint32_t);
	if (need > MOE_STATIC_SCRATCH_BYTES) {
		set_err("ffn_noalloc: T=%zu needs %zu bytes of scratch, beyond the %zu-byte "
			"static array", T, need, (size_t)MOE_STATIC_SCRATCH_BYTES);
		return 0;
	}
	uint32_t *ids = d_ids_out ? d_ids_out : (uint32_t *)(base + ids_off);
	float *w = d_w_out ? d_w_out : (float *)(base + ids_off + P * sizeof(uint32_t));
	L->used_static = 1;
	LCHK(moe_launch_fused(L->wtype, d_x, L->d_router, d_router_bias, L->d_gate, L->d_up,
			      L->d_down, L->gu_stride, L->down_stride, ids, w,
			      (uint64_t *)(base + part_off), d_out, (uint32_t *)base, (int)T,
			      (int)L->E, (int)L->EI, (int)L->NE, (int)L->topk, L->renorm,
			      L->fused_grid, L->spin, NULL, NULL, pick_stream(L, stream)),
	     "fused layer (static scratch)");
	return 1;
}

static int check_T(size_t T)
{
	if (T == 0 || T > 65535) {
		set_err("token count %zu out of range 1..65535", T);
		return 0;
	}
	return 1;
}

static int route(hip_moe_layer *L, const float *d_x, size_t T, const float *d_bias,
		 float *d_logits, float *d_probs, uint32_t *d_ids, float *d_w, void *d_xh,
		 hipStream_t s)
{
	LCHK(moe_launch_router(d_x, L->d_router, d_bias, d_logits, (int)T, (int)L->E,
			       (int)L->NE, s), "router");
	LCHK(moe_launch_softmax_topk(d_logits, d_probs, d_ids, d_w, (int)T, (int)L->NE,
				     (int)L->topk, L->renorm, d_x, d_xh, (int)L->E, s),
	     "softmax/top-k");
	return 1;
}

int hip_moe_route_dev(hip_moe_layer *L, const float *d_x, size_t T,
		      const float *d_router_bias, float *d_logits, float *d_probs,
		      uint32_t *d_ids, float *d_w, void *stream)
{
	if (!L || !d_x || !d_ids || !d_w) {
		set_err("route: NULL argument");
		return 0;
	}
	if (!check_T(T) || !ensure_scratch(L, T, pick_stream(L, stream)))
		return 0;
	return route(L, d_x, T, d_router_bias, d_logits ? d_logits : L->d_logits, d_probs,
		     d_ids, d_w, NULL, pick_stream(L, stream));
}

/* the path a call of T tokens takes (HIP_MOE_PATH_*), 0 if none applies */
static int choose_path(const hip_moe_layer *L, size_t T)
{
	/* K-quant experts: two launches (routing and gate/up, then down and
	 * combine) for a decode-sized call, else the per-pair products of
	 * kq_moe.hip */
	if (L->kq) {
		const int kdec = L->fused_grid > 0 &&
				 moe_kq_decode_supported(L->wtype, L->E, L->EI, L->NE, T, L->topk);
		switch (L->path) {
		case HIP_MOE_PATH_DECODE:
			return kdec ? HIP_MOE_PATH_DECODE : 0;
		case HIP_MOE_PATH_GEMV:
			return HIP_MOE_PATH_GEMV;
		case HIP_MOE_PATH_GROUPED:
			return 0;
		default:
			return kdec ? HIP_MOE_PATH_DECODE : HIP_MOE_PATH_GEMV;
		}
	}
	int dec = L->fused_grid > 0 &&
		  moe_fused_supported(L->wtype, L->E, L->EI, L->NE, T, L->topk);
	int grp = moe_prefill_supported(L->wtype, L->E, L->EI, L->NE) &&
		  moe_prefill_max_tiles(T * L->topk, L->NE) <= moe_prefill_tile_cap();
	switch (L->path) {
	case HIP_MOE_PATH_DECODE:
		return dec ? HIP_MOE_PATH_DECODE : 0;
	case HIP_MOE_PATH_GEMV:
		return HIP_MOE_PATH_GEMV;
	case HIP_MOE_PATH_GROUPED:
		return grp ? HIP_MOE_PATH_GROUPED : 0;
	default:
		/* one launch, but each (token, slot) streams its expert: taken while
		 * the pairs stay at 3/4 of the experts.  Measured crossings: OLMoE
		 * Q8_0 T=6 decode 85.0 / grouped 88.5 us, T=8 103.0 / 90.7;
		 * Mixtral Q4_0 T=3 141.0 / 163.6, T=4 168.2 / 163.6 */
		if (dec && 4 * T * L->topk <= 3 * L->NE)
			return HIP_MOE_PATH_DECODE;
		/* more pairs than experts: stream each touched expert once */
		if (grp)
			return HIP_MOE_PATH_GROUPED;
		return HIP_MOE_PATH_GEMV;
	}
}

int hip_moe_set_path(hip_moe_layer *L, int path)
{
	if (!L || path < HIP_MOE_PATH_AUTO || path > HIP_MOE_PATH_GROUPED) {
		set_err("set_path: bad layer or path %d", path);
		return 0;
	}
	L->path = path;
	return 1;
}

int hip_moe_path_for(const hip_moe_layer *L, size_t T)
{
	if (!L || T == 0)
		return 0;
	return choose_path(L, T);
}

/* the second launch of a decode-sized call on K-quant experts: down and
 * combine as one, or (longer d_ff) the per-pair down products and the
 * combine */
static int kq_decode_tail(hip_moe_layer *L, const uint32_t *ids, const float *w, float *d_out,
			  size_t T, hipStream_t s)
{
	if (moe_kq_down_combine_ok(T, L->topk, L->E, L->EI)) {
		LCHK(moe_launch_kq_down_combine(L->dtype, L->d_down, L->down_stride, ids, w, L->d_h,
						d_out, (int)T, (int)L->topk, (int)L->E, (int)L->EI,
						s),
		     "K-quant down + combine");
		return 1;
	}
	LCHK(moe_launch_kq_down(L->dtype, L->d_down, L->down_stride, ids, L->d_h, L->d_ypart,
				(int)(T * L->topk), (int)L->E, (int)L->EI, s),
	     "K-quant down");
	LCHK(moe_launch_combine(L->d_ypart, w, d_out, (int)T, (int)L->topk, (int)L->E, 1, s),
	     "combine");
	return 1;
}

int moe_norm_decode_ok(const hip_moe_layer *L)
{
	return L && choose_path(L, 1) == HIP_MOE_PATH_DECODE;
}

int moe_ffn_dev_norm(hip_moe_layer *L, const float *d_h, const float *d_norm_w, float *d_x_out,
		     float *d_out, uint32_t *d_ids_out, float *d_w_out, void *stream)
{
	if (!L || !d_h || !d_norm_w || !d_x_out || !d_out) {
		set_err("ffn_norm: NULL argument");
		return 0;
	}
	if (!moe_norm_decode_ok(L)) {
		set_err("ffn_norm: one token does not take the decode kernel on this layer");
		return 0;
	}
	hipStream_t s = pick_stream(L, stream);
	if (!ensure_scratch(L, 1, s))
		return 0;
	uint32_t *ids = d_ids_out ? d_ids_out : L->d_ids;
	float *w = d_w_out ? d_w_out : L->d_w;
	if (L->kq) {
		LCHK(moe_launch_kq_route_gateup(L->wtype, d_h, L->d_router, NULL, L->d_gate,
						L->d_up, L->gu_stride, ids, w, L->d_h, L->d_sync, 1,
						(int)L->E, (int)L->EI, (int)L->NE, (int)L->topk,
						L->renorm, L->fused_grid, L->spin, d_norm_w, d_x_out,
						s),
		     "K-quant routing + gate/up (normalising its input)");
		return kq_decode_tail(L, ids, w, d_out, 1, s);
	}
	LCHK(moe_launch_fused(L->wtype, d_h, L->d_router, NULL, L->d_gate, L->d_up, L->d_down,
			      L->gu_stride, L->down_stride, ids, w, L->d_part, d_out, L->d_sync, 1,
			      (int)L->E, (int)L->EI, (int)L->NE, (int)L->topk, L->renorm,
			      L->fused_grid, L->spin, d_norm_w, d_x_out, s),
	     "fused layer (normalising its input)");
	return 1;
}

int hip_moe_ffn_dev(hip_moe_layer *L, const float *d_x, float *d_out, size_t T,
		    const float *d_router_bias, uint32_t *d_ids_out, float *d_w_out,
		    void *stream)
{
	if (!L || !d_x || !d_out) {
		set_err("ffn: NULL argument");
		return 0;
	}
	hipStream_t s = pick_stream(L, stream);
	if (!check_T(T) || !ensure_scratch(L, T, s))
		return 0;
	uint32_t *ids = d_ids_out ? d_ids_out : L->d_ids;
	float *w = d_w_out ? d_w_out : L->d_w;
	int P = (int)(T * L->topk);
	int path = choose_path(L, T);

	if (!path) {
		set_err("ffn: the requested path does not apply to this layer and T=%zu", T);
		return 0;
	}
	if (path == HIP_MOE_PATH_DECODE && L->kq) {
		LCHK(moe_launch_kq_route_gateup(L->wtype, d_x, L->d_router, d_router_bias, L->d_gate,
						L->d_up, L->gu_stride, ids, w, L->d_h, L->d_sync,
						(int)T, (int)L->E, (int)L->EI, (int)L->NE,
						(int)L->topk, L->renorm, L->fused_grid, L->spin, NULL,
						NULL, s),
		     "K-quant routing + gate/up");
		return kq_decode_tail(L, ids, w, d_out, T, s);
	}
	if (path == HIP_MOE_PATH_DECODE) {
		LCHK(moe_launch_fused(L->wtype, d_x, L->d_router, d_router_bias, L->d_gate,
				      L->d_up, L->d_down, L->gu_stride, L->down_stride,
				      ids, w, L->d_part, d_out, L->d_sync,
				      (int)T, (int)L->E, (int)L->EI, (int)L->NE, (int)L->topk,
				      L->renorm, L->fused_grid, L->spin, NULL, NULL, s),
		     "fused layer");
		return 1;
	}
	if (!route(L, d_x, T, d_router_bias, L->d_logits, NULL, ids, w,
		   path == HIP_MOE_PATH_GROUPED ? L->d_xh : NULL, s))
		return 0;
	if (path == HIP_MOE_PATH_GROUPED) {
		int split = 1;
		LCHK(moe_launch_prefill(L->wtype, L->d_xh, L->d_gate_g, L->d_up_g, L->d_down,
					L->gu_stride, L->down_stride, ids, L->d_rows,
					L->d_tile_e, L->d_h16, L->d_ypart, (int)T, (int)L->topk,
					(int)L->E, (int)L->EI, (int)L->NE,
					(int)(L->ypart_cap / ((size_t)P * L->E)), &split, s),
		     "grouped GEMMs");
		LCHK(moe_launch_combine(L->d_ypart, w, d_out, (int)T, (int)L->topk, (int)L->E,
					split, s), "combine");
		return 1;
	}
	if (L->kq) {
		LCHK(moe_launch_kq_gateup(L->wtype, L->d_gate, L->d_up, L->gu_stride, ids, d_x,
					  L->d_h, P, (int)L->topk, (int)L->E, (int)L->EI, s),
		     "K-quant gate/up");
		LCHK(moe_launch_kq_down(L->dtype, L->d_down, L->down_stride, ids, L->d_h,
					L->d_ypart, P, (int)L->E, (int)L->EI, s),
		     "K-quant down");
		LCHK(moe_launch_combine(L->d_ypart, w, d_out, (int)T, (int)L->topk, (int)L->E, 1, s),
		     "combine");
		return 1;
	}
	LCHK(moe_launch_gateup(L->wtype, L->d_gate, L->d_up, L->gu_stride, ids, -1, d_x,
			       L->d_h, P, (int)L->topk, (int)L->E, (int)L->EI, s),
	     "gate/up");
	int kch = 1;
	LCHK(moe_launch_down(L->wtype, L->d_down, L->down_stride, ids, -1, L->d_h,
			     L->d_ypart, L->ypart_cap, P, (int)L->E, (int)L->EI, &kch, s),
	     "down");
	LCHK(moe_launch_combine(L->d_ypart, w, d_out, (int)T, (int)L->topk, (int)L->E, kch, s),
	     "combine");
	return 1;
}

int hip_moe_expert_ffn_dev(hip_moe_layer *L, size_t expert, const float *d_x,
			   float *d_out, void *stream)
{
	if (!L || !d_x || !d_out) {
		set_err("expert_ffn: NULL argument");
		return 0;
	}
	if (expert >= L->NE) {
		set_err("expert_ffn: expert %zu >= NE %zu", expert, L->NE);
		return 0;
	}
	hipStream_t s = pick_stream(L, stream);
	if (!ensure_scratch(L, 1, s))
		return 0;
	if (L->kq) {
		/* the kernels take the expert from an id list: one entry */
		const uint32_t id = (uint32_t)expert;
		/* ordered after the stream's earlier users of d_ids; the source
		 * lives on this stack frame, so the copy completes here */
		HIPCHK(hipMemcpyAsync(L->d_ids, &id, sizeof(id), hipMemcpyHostToDevice, s),
		       "copy expert id");
		HIPCHK(hipStreamSynchronize(s), "synchronize");
		LCHK(moe_launch_kq_gateup(L->wtype, L->d_gate, L->d_up, L->gu_stride, L->d_ids,
					  d_x, L->d_h, 1, 1, (int)L->E, (int)L->EI, s),
		     "K-quant gate/up");
		LCHK(moe_launch_kq_down(L->dtype, L->d_down, L->down_stride, L->d_ids, L->d_h,
					L->d_ypart, 1, (int)L->E, (int)L->EI, s),
		     "K-quant down");
		LCHK(moe_launch_combine(L->d_ypart, NULL, d_out, 1, 1, (int)L->E, 1, s), "combine");
		return 1;
	}
	LCHK(moe_launch_gateup(L->wtype, L->d_gate, L->d_up, L->gu_stride, NULL, (int)expert,
			       d_x, L->d_h, 1, 1, (int)L->E, (int)L->EI, s), "gate/up");
	int kch = 1;
	LCHK(moe_launch_down(L->wtype, L->d_down, L->down_stride, NULL, (int)expert, L->d_h,
			     L->d_ypart, L->ypart_cap, 1, (int)L->E, (int)L->EI, &kch, s),
	     "down");
	LCHK(moe_launch_combine(L->d_ypart, NULL, d_out, 1, 1, (int)L->E, kch, s), "combine");
	return 1;
fail:
	return 0;
}

static int ensure_io(hip_moe_layer *L, size_t T)
{
	if (T <= L->cap_io)
		return 1;
	hipFree(L->d_x);
	hipFree(L->d_out);
	hipFree(L->d_bias);
	hipFree(L->d_ids_io);
	hipFree(L->d_w_io);
	L->d_x = L->d_out = L->d_bias = L->d_w_io = NULL;
	L->d_ids_io = NULL;
	L->cap_io = 0;
	HIPCHK(hipMalloc((void **)&L->d_x, T * L->E * sizeof(float)), "hipMalloc(x)");
	HIPCHK(hipMalloc((void **)&L->d_out, T * L->E * sizeof(float)), "hipMalloc(out)");
	HIPCHK(hipMalloc((void **)&L->d_bias, L->NE * sizeof(float)), "hipMalloc(bias)");
	HIPCHK(hipMalloc((void **)&L->d_ids_io, T * L->topk * sizeof(uint32_t)),
	       "hipMalloc(ids)");
	HIPCHK(hipMalloc((void **)&L->d_w_io, T * L->topk * sizeof(float)), "hipMalloc(w)");
	L->cap_io = T;
	return 1;
fail:
	return 0;
}

int hip_moe_ffn(hip_moe_layer *L, const float *x, float *out, size_t T,
		const float *router_bias, uint32_t *ids_out, float *w_out)
{
	if (!L || !x || !out) {
		set_err("ffn: NULL argument");
		return 0;
	}
	if (!check_T(T) || !ensure_io(L, T))
		return 0;
	hipStream_t s = L->stream;
	HIPCHK(hipMemcpyAsync(L->d_x, x, T * L->E * sizeof(float), hipMemcpyHostToDevice, s),
	       "copy x");
	if (router_bias)
		HIPCHK(hipMemcpyAsync(L->d_bias, router_bias, L->NE * sizeof(float),
				      hipMemcpyHostToDevice, s), "copy bias");
	if (!hip_moe_ffn_dev(L, L->d_x, L->d_out, T, router_bias ? L->d_bias : NULL,
			     L->d_ids_io, L->d_w_io, s))
		return 0;
	HIPCHK(hipMemcpyAsync(out, L->d_out, T * L->E * sizeof(float), hipMemcpyDeviceToHost, s),
	       "copy out");
	if (ids_out)
		HIPCHK(hipMemcpyAsync(ids_out, L->d_ids_io, T * L->topk * sizeof(uint32_t),
				      hipMemcpyDeviceToHost, s), "copy ids");
	if (w_out)
		HIPCHK(hipMemcpyAsync(w_out, L->d_w_io, T * L->topk * sizeof(float),
				      hipMemcpyDeviceToHost, s), "copy w");
	/* a bounded wait inside the decode kernel ran out: report and reset */
	if (check_and_reset(L, s) != 0)
		return 0;
	return 1;
fail:
	return 0;
}

int hip_moe_expf_dev(const float *d_in, float *d_out, size_t n, void *stream)
{
	LCHK(moe_launch_expf(d_in, d_out, n, stream), "expf");
	return 1;
}

int hip_moe_copy_dev(const void *d_src, void *d_dst, size_t bytes, void *stream)
{
	if (bytes == 0 || bytes % 16) {
		set_err("hip_moe_copy_dev: bytes must be a positive multiple of 16");
		return 0;
	}
	LCHK(moe_launch_copy(d_src, d_dst, bytes, stream), "copy");
	return 1;
}

/* ------------------------------------------------------------------ */
/* dense quantized matrices (tensor_mma_transposed_2x2 on Q8_0/Q4_0)   */
/* ------------------------------------------------------------------ */

struct hip_moe_qmat {
	int wtype, device;
	size_t N, K, bytes;
	uint8_t *d_w;       /* the GGUF blocks, row-major, unchanged */
	hipStream_t stream; /* the device's shared library stream */
	int grid1, grid;    /* workgroups for T == 1 and T > 1 (moe_qgemv_grid) */
	/* the partial sums of the matrix-core product (T > 1), for up to
	 * split_T tokens; calls that overlap on one matrix race on them */
	void *d_split;
	size_t split_T;
	int qmm;            /* K suits the matrix-core product */
	/* staging for the host-pointer entry point */
	size_t cap_T;
	float *d_x, *d_add, *d_out;
};

/* tokens the matrix-core product's split buffer holds from upload on (the
 * device entry point allocates nothing: more tokens take the per-token
 * product) */
#define QMAT_SPLIT_T 64

/* the matrix-core product's partial sums for up to T tokens (the old ones
 * freed first) */
static int qmat_split_alloc(hip_moe_qmat *W, size_t T)
{
	hipFree(W->d_split);
	W->d_split = NULL;
	W->split_T = 0;
	const size_t wb = moe_qmm_work_bytes((int)T, (int)W->N, (int)W->K);
	if (wb)
		HIPCHK(hipMalloc(&W->d_split, wb), "hipMalloc(qmat partial sums)");
	W->split_T = T;
	return 1;
fail:
	return 0;
}

hip_moe_qmat *hip_moe_qmat_upload(const void *qdata, int wtype, size_t N, size_t K)
{
	hip_moe_qmat *W = NULL;
	int ndev = 0;

	if (wtype != HIP_MOE_Q8_0 && wtype != HIP_MOE_Q4_0 && !is_kquant(wtype)) {
		set_err("qmat_upload: unsupported weight type %d (Q8_0=1, Q4_0=2, Q4_K=3, "
			"Q6_K=5)", wtype);
		return NULL;
	}
	if (!qdata) {
		set_err("qmat_upload: NULL weight pointer");
		return NULL;
	}
	if (is_kquant(wtype)) {
		/* a thread per 256-value super-block; the tokens' Q8_K blocks in LDS */
		if (N == 0 || N > 0x7fffffff || K > 0x7fffffff || !moe_kq_supported(wtype, (int)K)) {
			set_err("qmat_upload: N=%zu K=%zu not supported for K-quants (N >= 1, K a "
				"multiple of 256 up to 32768)", N, K);
			return NULL;
		}
	} else if (N == 0 || N > 0x7fffffff || K < 256 || K % 256 ||
		   !is_pow2(K / MOE_SEG_COLS) || K / MOE_SEG_COLS > 64) {
		/* one wave of K/64 lanes covers a row, no K-split */
		set_err("qmat_upload: N=%zu K=%zu not supported (N >= 1, K/64 a power of two "
			"4..64)", N, K);
		return NULL;
	}
	if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
		set_err("qmat_upload: no HIP device");
		return NULL;
	}
	W = calloc(1, sizeof(*W));
	if (!W) {
		set_err("qmat_upload: out of host memory");
		return NULL;
	}
	W->wtype = wtype;
	W->N = N;
	W->K = K;
	W->bytes = N * row_bytes(wtype, K);
	HIPCHK(hipGetDevice(&W->device), "hipGetDevice");
	W->stream = device_stream(W->device);
	if (!W->stream)
		goto fail;
	/* resident workgroups, queried here rather than at a call that may be
	 * under graph capture */
	if (is_kquant(wtype)) {
		W->grid1 = moe_kq_grid(wtype, (int)K, 1);
		W->grid = moe_kq_grid(wtype, (int)K, 8);
	} else {
		W->grid1 = moe_qgemv_grid(wtype, (int)K, 1);
		W->grid = moe_qgemv_grid(wtype, (int)K, 0);
	}
	W->qmm = !is_kquant(wtype) && moe_qmm_supported(wtype, (int)K);
	if (W->qmm && !qmat_split_alloc(W, QMAT_SPLIT_T))
		goto fail;
	/* the K-quant loads read up to MOE_KQ_SLACK bytes past the last block */
	HIPCHK(hipMalloc((void **)&W->d_w, W->bytes + MOE_KQ_SLACK), "hipMalloc(qmat)");
	HIPCHK(hipMemset(W->d_w + W->bytes, 0, MOE_KQ_SLACK), "clear qmat slack");
	HIPCHK(hipMemcpy(W->d_w, qdata, W->bytes, hipMemcpyHostToDevice), "upload qmat");
	return W;
fail:
	hip_moe_qmat_free(W);
	return NULL;
}

/* mma_init (matmul.c:13-33): add holds T*N values (copied) or N (every row) */
static int check_add(const hip_moe_qmat *W, size_t T, const float *add, size_t add_len)
{
	if (add && add_len != W->N && add_len != T * W->N) {
		set_err("qmat_mul: add holds %zu values, not N=%zu or T*N=%zu", add_len, W->N,
			T * W->N);
		return 0;
	}
	return 1;
}

int hip_moe_qmat_mul_dev(const hip_moe_qmat *W, const float *d_x, size_t T,
			 const float *d_add, size_t add_len, float *d_out, void *stream)
{
	if (!W || !d_x || !d_out) {
		set_err("qmat_mul: NULL argument");
		return 0;
	}
	if (T == 0 || T > 65535 || T * W->N > ((size_t)1 << 40)) {
		set_err("qmat_mul: token count %zu out of range 1..65535", T);
		return 0;
	}
	if ((uintptr_t)d_x % 16) {
		set_err("qmat_mul: x must be 16-byte aligned");
		return 0;
	}
	if (!check_add(W, T, d_add, add_len))
		return 0;
	void *s = stream ? stream : (void *)W->stream;
	if (is_kquant(W->wtype)) {
		LCHK(moe_launch_kq_gemv(W->wtype, W->d_w, (int)W->N, (int)W->K, d_x, (int)T, d_add,
					add_len == T * W->N, d_out, T == 1 ? W->grid1 : W->grid, s),
		     "kq_gemv");
	} else if (T > 1 && W->qmm && T <= W->split_T) {
		/* several tokens: on the matrix cores, at fp32 accuracy */
		LCHK(moe_launch_qmm(W->wtype, W->d_w, (int)W->N, (int)W->K, d_x, (int)T, d_add,
				    add_len == T * W->N, d_out, W->d_split, s), "qmm");
	} else
		LCHK(moe_launch_qgemv(W->wtype, W->d_w, (int)W->N, (int)W->K, d_x, (int)T, d_add,
				      add_len == T * W->N, d_out, T == 1 ? W->grid1 : W->grid, s),
		     "qgemv");
	return 1;
}

int hip_moe_qmat_mul(hip_moe_qmat *W, const float *x, size_t T, const float *add,
		     size_t add_len, float *out)
{
	if (!W || !x || !out) {
		set_err("qmat_mul: NULL argument");
		return 0;
	}
	if (T == 0 || T > 65535) {
		set_err("qmat_mul: token count %zu out of range 1..65535", T);
		return 0;
	}
	if (!check_add(W, T, add, add_len))
		return 0;
	hipStream_t s = W->stream;
	if (T > W->cap_T) {
		hipFree(W->d_x);
		hipFree(W->d_add);
		hipFree(W->d_out);
		W->d_x = W->d_add = W->d_out = NULL;
		W->cap_T = 0;
		HIPCHK(hipMalloc((void **)&W->d_x, T * W->K * sizeof(float)), "hipMalloc(x)");
		HIPCHK(hipMalloc((void **)&W->d_add, T * W->N * sizeof(float)), "hipMalloc(add)");
		HIPCHK(hipMalloc((void **)&W->d_out, T * W->N * sizeof(float)), "hipMalloc(out)");
		W->cap_T = T;
	}
	if (W->qmm && T > W->split_T) { /* the host entry point may allocate */
		/* device-pointer calls on any stream may still read the old buffer */
		HIPCHK(hipDeviceSynchronize(), "synchronize");
		if (!qmat_split_alloc(W, T))
			return 0;
	}
	HIPCHK(hipMemcpyAsync(W->d_x, x, T * W->K * sizeof(float), hipMemcpyHostToDevice, s),
	       "copy x");
	if (add)
		HIPCHK(hipMemcpyAsync(W->d_add, add, add_len * sizeof(float),
				      hipMemcpyHostToDevice, s), "copy add");
	if (!hip_moe_qmat_mul_dev(W, W->d_x, T, add ? W->d_add : NULL, add_len, W->d_out, s))
		return 0;
	HIPCHK(hipMemcpyAsync(out, W->d_out, T * W->N * sizeof(float), hipMemcpyDeviceToHost, s),
	       "copy out");
	HIPCHK(hipStreamSynchronize(s), "synchronize");
	return 1;
fail:
	return 0;
}

size_t hip_moe_qmat_bytes(const hip_moe_qmat *W)
{
	return W ? W->bytes : 0;
}

void hip_moe_qmat_free(hip_moe_qmat *W)
{
	if (!W)
		return;
	hipFree(W->d_w);
	hipFree(W->d_split);
	hipFree(W->d_x);
	hipFree(W->d_add);
	hipFree(W->d_out);
	free(W); /* W->stream is the device's shared stream: it stays */
}

int hip_moe_quantize_q8k_dev(const float *d_x, size_t T, size_t K, float *d_d, int8_t *d_qs,
			     int16_t *d_bsums, void *stream)
{
	if (!d_x || !d_d || !d_qs || !d_bsums) {
		set_err("quantize_q8k: NULL argument");
		return 0;
	}
	if (T == 0 || K == 0 || K % 256 || T * K > ((size_t)1 << 31)) {
		set_err("quantize_q8k: T=%zu K=%zu not supported (K a multiple of 256, T*K < 2^31)",
			T, K);
		return 0;
	}
	if ((uintptr_t)d_x % 16 || (uintptr_t)d_qs % 4) {
		set_err("quantize_q8k: x must be 16-byte and qs 4-byte aligned");
		return 0;
	}
	int dev = 0;
	if (hipGetDevice(&dev) != hipSuccess) {
		set_err("quantize_q8k: no HIP device");
		return 0;
	}
	hipStream_t s = stream ? (hipStream_t)stream : device_stream(dev);
	LCHK(moe_launch_q8k_quantize(d_x, (int)T, (int)K, d_d, d_qs, d_bsums, s), "q8k_quantize");
	return 1;
}
