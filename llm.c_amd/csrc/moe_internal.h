/*
 * Internal interface between the C host layer (hip_moe.c) and the HIP
 * kernels (moe_kernels.hip).  Every launcher returns a hipError_t value
 * (0 = success) and enqueues on the given stream without waiting.
 */
#ifndef MOE_INTERNAL_H
#define MOE_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry shared by host and kernels. */
#define MOE_QK 32           /* elements per block */
#define MOE_SEG_COLS 64     /* columns one lane holds: a pair of blocks */
#define MOE_MAX_NE 256
/* Gate and up matrices are stored in groups of MOE_GU_GROUP rows; inside a
 * group, piece-major: for piece s (GGML blocks 2s and 2s+1, 64 columns) the
 * pieces of the group's rows follow each other.  A decode item (32 rows of
 * d_ff) is then one contiguous run, and a K-step of the grouped GEMMs reads
 * one contiguous run per group. */
#define MOE_GU_GROUP 32
#define MOE_MAX_TOPK 64
#define MOE_FUSED_MAX_P 64  /* T*K handled by the persistent decode kernel */
#define MOE_SYNC_ERR_WORD 256 /* error word in the persistent kernel's counters: */
#define MOE_ERR_ROUTE 1   /* a wait for router logits ran out */
#define MOE_ERR_COMBINE 2 /* a wait for partial sums ran out */
#define MOE_ERR_FLAGS 3   /* the end-of-launch start-flag check ran out */
#define MOE_SPIN_DEFAULT (1 << 20) /* poll rounds before a decode-kernel wait gives up */

/* lanes per gate/up row for a K-long dot: the largest power of two <= 64
 * that divides K / 64, and the number of K-chunks the row is split into. */
int moe_lanes_per_row(size_t K);
int moe_kchunks(size_t K);

int moe_launch_router(const float *x, const float *wr, const float *bias,
                      float *logits, int T, int E, int NE, void *stream);

/* xh (optional, f16 [T][E]): also write the tokens x [T][E] rounded to f16 */
int moe_launch_softmax_topk(const float *logits, float *probs, uint32_t *ids,
                            float *w, int T, int NE, int K, int renorm,
                            const float *x, void *xh, int E, void *stream);

/* h[p][EI] = silu(gate_e . x_t) * (up_e . x_t), p = t*K + s, e = ids[p]
 * (or fixed_e >= 0 for every p). */
int moe_launch_gateup(int wtype, const uint8_t *gate, const uint8_t *up,
                      size_t expert_stride, const uint32_t *ids, int fixed_e,
                      const float *x, float *h, int P, int K, int E, int EI,
                      void *stream);

/* Down matrices are stored as EI/32 panels of E blocks each (panel c holds
 * block c of every row).  ypart[p][kc][E] = partial dots of down_e rows
 * with h[p] over K-chunk kc, *kchunks chunks, at most ypart_cap floats. */
int moe_launch_down(int wtype, const uint8_t *down, size_t expert_stride,
                    const uint32_t *ids, int fixed_e, const float *h,
                    float *ypart, size_t ypart_cap, int P, int E, int EI, int *kchunks,
                    void *stream);
/* out[t][j] = (add ? add[add_rows ? t*N + j : j] : 0) + dot(x[t], W row j),
 * W of N rows of K columns in Q8_0 (wtype 1) or Q4_0 (2) blocks; K/64 a
 * power of two 4..64; x 16-byte aligned (moe_qgemv.hip).  nwg workgroups
 * (moe_qgemv_grid; <= 0: a fixed default). */
int moe_launch_qgemv(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
                     const float *add, int add_rows, float *out, int nwg, void *stream);
/* workgroups the device holds at once for the (wtype, K, T == 1) instance */
int moe_qgemv_grid(int wtype, int K, int one);

/* the same product for several tokens on the matrix cores at fp32
 * accuracy (moe_qmm.hip): x [T][K] fp32, 16-byte aligned; K = 256, 512
 * or a multiple of 512 (moe_qmm_supported); work holds
 * moe_qmm_work_bytes(T, N, K) bytes (none for K <= 512) */
int moe_qmm_supported(int wtype, int K);
size_t moe_qmm_work_bytes(int T, int N, int K);
int moe_launch_qmm(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
                   const float *add, int add_rows, float *out, void *work, void *stream);
/* moe_qmm_stretches: the KS column stretches a product of K columns splits
 * into; moe_launch_qmm_parts (KS > 1): only the KS partial sums, slices of
 * T * N floats in work, for the caller to add in stretch order */
int moe_qmm_stretches(int K);
int moe_launch_qmm_parts(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
                         void *work, void *stream);

/* The same product on a Q4_K (wtype 3) or Q6_K (5) matrix through Q8_K
 * activations, bit for bit the reference's (kquant.hip); the matrix buffer
 * needs MOE_KQ_SLACK bytes past its end.  moe_kq_supported: K a multiple of
 * 256 whose staging fits in LDS. */
#define MOE_KQ_SLACK 16
int moe_kq_supported(int wtype, int K);
int moe_kq_grid(int wtype, int K, int T);
int moe_launch_kq_gemv(int wtype, const uint8_t *W, int N, int K, const float *x, int T,
                       const float *add, int add_rows, float *out, int nwg, void *stream);
/* The same product for one token whose input is rms_norm(a + b) * w (b may
 * be NULL), normalised in every workgroup with the row norm kernel's
 * arithmetic (the same bits); workgroup 0 writes a + b to h_out and the
 * normalised token to x_out (either may be NULL).  moe_kq_norm_ok: whether
 * this form takes wtype at K (the register path, K <= 4096). */
int moe_kq_norm_ok(int wtype, int K);
int moe_launch_kq_gemv_norm(int wtype, const uint8_t *W, int N, int K, const float *a,
                            const float *b, const float *w, float *h_out, float *x_out,
                            float *out, int nwg, void *stream);
/* The expert products of a MoE layer with K-quant experts (kq_moe.hip):
 * gate/up type gt, down type dt (3 = Q4_K, 5 = Q6_K), bit for bit the
 * reference's fused_ffn_silu; y [P][E] goes to moe_launch_combine with one
 * chunk. */
int moe_kq_layer_supported(int gt, int dt, size_t E, size_t EI);
int moe_launch_kq_gateup(int gt, const uint8_t *gate, const uint8_t *up, size_t gu_stride,
                         const uint32_t *ids, const float *x, float *h, int P, int K, int E,
                         int EI, void *stream);
int moe_launch_kq_down(int dt, const uint8_t *down, size_t dn_stride, const uint32_t *ids,
                       const float *h, float *y, int P, int E, int EI, void *stream);
/* The decode-sized K-quant layer: routing and gate/up in one launch
 * (moe_decode.hip: one workgroup per CU, the decode kernel's sync words)
 * writing h [P][EI], ids and weights; then the down dots and the combine
 * into out in one launch where d_ff is at most 1024 (kq_moe.hip), else
 * moe_launch_kq_down and moe_launch_combine.  The same arithmetic as the
 * kernels above. */
int moe_kq_decode_supported(int gt, size_t E, size_t EI, size_t NE, size_t T, size_t K);
int moe_kq_decode_grid(int gt, size_t E, size_t NE);
int moe_launch_kq_route_gateup(int gt, const float *x, const float *router, const float *bias,
                               const uint8_t *gate, const uint8_t *up, size_t gu_stride,
                               uint32_t *ids, float *w, float *h, uint32_t *sync, int T, int E,
                               int EI, int NE, int K, int renorm, int grid, int spin,
                               const float *norm_w, float *x_out, void *stream);
int moe_kq_down_combine_ok(size_t T, size_t K, size_t E, size_t EI);
int moe_launch_kq_down_combine(int dt, const uint8_t *down, size_t dn_stride,
                               const uint32_t *ids, const float *w, const float *h, float *out,
                               int T, int K, int E, int EI, void *stream);
/* quantize_row_q8 of T rows of K values: d[T][K/256], qs[T][K], bsums[T][K/256][16] */
int moe_launch_q8k_quantize(const float *x, int T, int K, float *d, int8_t *qs,
                            int16_t *bsums, void *stream);

/* ypart floats moe_launch_down may use for any pair count up to P */
size_t moe_down_part_floats(size_t E, size_t EI, size_t P);

/* out[t][E] = sum over slots s, in order, of y[t*K+s] / (1/w[t*K+s]);
 * y = sum of the kchunks partials in order.  w == NULL means weight 1. */
int moe_launch_combine(const float *ypart, const float *w, float *out, int T,
                       int K, int E, int kchunks, void *stream);

int moe_launch_expf(const float *in, float *out, size_t n, void *stream);
int moe_launch_copy(const void *src, void *dst, size_t bytes, void *stream);

/* Grouped path (moe_prefill.hip): sort by expert + f16 MFMA GEMMs. */
#define MOE_WEIGHT_SLACK 256 /* bytes readable past the last weight row */
int moe_prefill_supported(int wtype, size_t E, size_t EI, size_t NE);
/* tile-table entries and sorted rows any call of at most P pairs uses */
int moe_prefill_max_tiles(size_t P, size_t NE);
size_t moe_prefill_max_rows(size_t P, size_t NE);
size_t moe_prefill_tile_ints(size_t P, size_t NE);
int moe_prefill_tile_cap(void);
/* ypart[p][split][E] for every pair p, *split (<= max_split) K-splits of
 * the down projection; combine with kchunks = *split */
int moe_launch_prefill(int wtype, const void *xh, const uint8_t *gate, const uint8_t *up,
                       const uint8_t *down, size_t gu_stride, size_t dn_stride,
                       const uint32_t *ids, int *rows, int *tile_e, void *h16, float *ypart,
                       int T, int K, int E, int EI, int NE, int max_split, int *split,
                       void *stream);

/* One-launch decode layer (moe_decode.hip) for T*K <= MOE_FUSED_MAX_P:
 * grid = one workgroup per CU (0: not applicable), sync words and tagged
 * 64-bit partial words it needs for T tokens. */
int moe_fused_supported(int wtype, size_t E, size_t EI, size_t NE, size_t T, size_t K);
int moe_fused_grid(int wtype, size_t E, size_t EI, size_t NE);
size_t moe_fused_sync_words(size_t T, size_t NE, int grid);
size_t moe_fused_part_words(size_t T, size_t K, size_t E, size_t EI, int grid);
int moe_launch_fused(int wtype, const float *x, const float *router, const float *bias,
                     const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                     size_t gu_stride, size_t dn_stride, uint32_t *ids, float *w,
                     uint64_t *part, float *out, uint32_t *sync, int T, int E, int EI, int NE,
                     int K, int renorm, int grid, int spin, const float *norm_w, float *x_out,
                     void *stream);

/* One token through the decode kernel with the layer's input normalised in
 * the launch: x = rms_norm(d_h) * d_norm_w (the one-token model kernels'
 * arithmetic; also written to d_x_out), then the layer on x, as
 * hip_moe_ffn_dev(L, x, d_out, 1, NULL, ids, w).  moe_norm_decode_ok: whether
 * one token takes the decode path on L (Q8_0/Q4_0 experts: k_moe_decode,
 * whose norm sums as the output product's gather; K-quant experts:
 * k_kq_route_gateup, whose norm sums as the row norm kernel). */
struct hip_moe_layer;
int moe_norm_decode_ok(const struct hip_moe_layer *L);
int moe_ffn_dev_norm(struct hip_moe_layer *L, const float *d_h, const float *d_norm_w,
                     float *d_x_out, float *d_out, uint32_t *d_ids_out, float *d_w_out,
                     void *stream);

/* How many times the layer's scratch was (re)allocated: a HIP graph that
 * was captured at another count names freed buffers and must be dropped. */
struct hip_moe_layer;
unsigned moe_scratch_gen(const struct hip_moe_layer *L);

/* Record an error message for hip_moe_last_error (and print it). */
void moe_set_error(const char *msg);

/* Static device scratch of the allocation-free decode entry point
 * (moe_decode.hip): MOE_STATIC_SCRATCH_BYTES per device, looked up and
 * cleared once per device by moe_static_scratch_setup (with that device
 * current), then addressed through moe_static_scratch(dev) only. */
#define MOE_STATIC_SCRATCH_BYTES ((size_t)12 << 20)
int moe_static_scratch_setup(int dev);
void *moe_static_scratch(int dev);

#ifdef __cplusplus
}
#endif
#endif
