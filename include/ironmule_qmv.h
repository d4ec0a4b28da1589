/*
 * ironmule_qmv.h — C ABI of the MI355X (gfx950) 4-bit affine group-quantised
 * matrix-vector product ("qmv") library, libironmule_qmv.so.
 *
 * Weight format (the reference's, unchanged, so callers pass their buffers as-is):
 *   w       uint32 (N, K/8), eight 4-bit values per word, low nibble first
 *           (element j of word u is (u >> 4j) & 0xF)
 *   scales  bf16 bit patterns (N, K/64), biases bf16 bit patterns (N, K/64)
 *   weight  scale * q + bias, q in 0..15, group size 64, bits 4
 *   x       bf16 (M, K) activation rows; y (M, N) bf16 or fp32
 *
 * Contract shared by every entry point:
 *   - all array pointers are device pointers; the caller allocates them;
 *   - the library never allocates, frees or synchronises per call; work is queued on
 *     `stream` (a hipStream_t, NULL for the default stream) and the call returns;
 *   - every output element is written exactly once (outputs need no initialisation);
 *   - the library keeps no state between calls and is reentrant; per-device set-up
 *     (architecture check, kernel attributes) happens once, on first use;
 *   - errors are returned as codes, never raised; imq_last_error() describes the last
 *     one on the calling thread.
 *
 * Alignment: w and every x row 16-byte aligned, ldx a multiple of 8 elements; scales,
 * biases 2-byte aligned; y 2-byte (bf16) or 4-byte (fp32) aligned.
 */
#ifndef IRONMULE_QMV_H
#define IRONMULE_QMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IMQ_ABI_VERSION 1

#ifndef IMQ_API
#define IMQ_API __attribute__((visibility("default")))
#endif

/* Return codes. */
#define IMQ_OK 0
#define IMQ_EINVAL 1       /* bad pointer, shape, stride, alignment or dtype code */
#define IMQ_EUNSUPPORTED 2 /* well-formed but outside the kernels: bits != 4, gs != 64, M > 32 */
#define IMQ_EUNAVAILABLE 3 /* no HIP device, or the current device is not gfx950 */
#define IMQ_ELAUNCH 6      /* the HIP runtime refused the launch */

/* Output dtype codes. */
#define IMQ_BF16 0
#define IMQ_F32 1
#define IMQ_F16 2 /* imq_dequant only */

/* Largest number of activation rows one call serves with a single weight sweep. */
#define IMQ_MAX_ROWS 32

/* Largest number of weights one imq_qmv_grouped call serves. */
#define IMQ_MAX_PROBLEMS 8

/* One weight and its activation/output rows, for imq_qmv_grouped. */
typedef struct imq_problem {
  const uint32_t* w;       /* (N, K/8) packed words */
  const uint16_t* scales;  /* (N, K/64) bf16 */
  const uint16_t* biases;  /* (N, K/64) bf16 */
  const uint16_t* x;       /* (M, K) bf16, rows ldx elements apart */
  int64_t ldx;
  void* y;                 /* (M, N) bf16 or fp32, rows ldy elements apart */
  int64_t ldy;
  int32_t N;
  int32_t K;
} imq_problem;

/* The ABI version this library implements (IMQ_ABI_VERSION). */
IMQ_API int32_t imq_abi_version(void);

/* IMQ_OK if the current HIP device is a gfx950 the kernels run on.  Fills `arch`
 * (NUL-terminated, may be NULL) and `cu_count` (may be NULL). */
IMQ_API int32_t imq_device_check(char* arch, size_t arch_len, int32_t* cu_count);

/*
 * y[m][n] = sum_k (scales[n][k/64] * q[n][k] + biases[n][k/64]) * x[m][k]
 * for m < M (1..32), n < N, with fp32 accumulation; y rounded to bf16 (nearest even)
 * or stored as fp32 per y_dtype.  The weight is read from memory once for all M rows
 * (the shared-weight multi-request form).
 *
 * Replaces the reference's per-call kernel launches of the 4-bit qmv:
 *   ironmule/qmv_k3840.py:299-310        run(kernel, w, scales, biases, x, N, K)  (M = 1)
 *   ironmule/qmv_variant.py:116-129      GatedVariantLinear.__call__ kernel branch (M = 1)
 *   ironmule/cuda_native.py:155-168      _qmv(x, w, scales, biases)              (M <= 8)
 *   ironmule/cuda_native.py:171-179      matmul(...) decode branch, LM head via
 *                                         NativeQuantizedEmbedding.as_linear (227-229)
 * x rows are `ldx` elements apart, y rows `ldy` elements apart.
 */
IMQ_API int32_t imq_qmv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                const uint16_t* x, int64_t ldx, void* y, int64_t ldy, int32_t M, int32_t N,
                int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype, void* stream);

/*
 * The gate and up projections of a SwiGLU MLP and their product, one launch:
 *   act[m][n] = bf16(silu(g) * u),  g = bf16(sum_k x[m][k] W_gate[n][k]),
 *                                   u = bf16(sum_k x[m][k] W_up[n][k]),
 * the bits of imq_qmv_grouped over (gate, up) at the same M followed by imq_silu_mul.
 * gate and up are N x K weights of the format above sharing x (M rows, `ldx` apart); act
 * rows are `ld_act` apart.  5 <= M <= 32 and K % 256 == 0, else IMQ_EUNSUPPORTED (the caller
 * makes the two launches).  Replaces the fused gate/up launch and the SwiGLU that follows it:
 *   ironmule/fast.py:186-215             fuse_projections (gate and up in one launch)
 *   ironmule/dense_plan.py:360            silu(gate) * up
 */
IMQ_API int32_t imq_qmv_gate_up_silu(const uint32_t* w_gate, const uint16_t* s_gate,
                const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up,
                const uint16_t* b_up, const uint16_t* x, int64_t ldx, uint16_t* act,
                int64_t ld_act, int32_t M, int32_t N, int32_t K, int32_t group_size,
                int32_t bits, void* stream);

/*
 * An RMSNorm folded into the projections around it (decode glue).  With
 * inv_m = 1 / sqrt(sum_n h[m][n]^2 / dim + eps), rms_norm(h) W^T = inv * ((h * w) W^T) row by
 * row, so the kernel that produces the residual stream h writes x' = bf16(h * w) and per
 * 64-column tile of h each row's partial sum of squares, and the projection that reads x'
 * scales its output rows by inv: the RMSNorm needs no launch of its own.  The rounding
 * points differ from bf16(bf16(h * inv) * w) by the place of one bf16 rounding.
 * Replaces the RMSNorm launches between the projections of the reference's decode step,
 * ironmule/dense_plan.py:348 and 359 (the input and post-attention norms).
 */
typedef struct imq_norm_in {
  const float* ssq;  /* row m's partial sums at ssq[m * ld + t], t < tiles; 16-byte aligned */
  int32_t tiles;     /* 1..128 partials per row, added in a fixed order */
  int32_t ld;        /* a multiple of 4, >= tiles */
  int32_t dim;       /* h's row length, the mean's divisor */
  float eps;
} imq_norm_in;

typedef struct imq_residual_out {
  float* h;                /* (M, N) fp32 residual rows, ldh apart: h += bf16(y) */
  int64_t ldh;
  const uint16_t* weight;  /* (N) bf16 weight of the next RMSNorm; NULL: update h only */
  uint16_t* x;             /* (M, N) bf16 x' = bf16(h * weight), rows ldx apart */
  int64_t ldx;             /* or IMQ_LD_TILED: x' in the 32-row tile layout (N % 64 == 0) */
  float* ssq;              /* NULL, or (M, ld): ssq[m * ld + t] = sum of h[m][n]^2 over
                            * the 64 columns n of tile t, t < ceil(N / 64) */
  int32_t ld;              /* a multiple of 4, >= ceil(N / 64) */
} imq_residual_out;

/* Bytes of workspace imq_qmv_norm needs for these problems at M rows (zero-filled before
 * its first use, left ready by every call, as for imq_qmv_grouped_ws). */
IMQ_API size_t imq_qmv_norm_workspace(const imq_problem* problems, int32_t count, int32_t M);

/*
 * imq_qmv_grouped_ws (bf16 outputs) with the RMSNorm of the inputs and/or the residual add
 * of the output folded in.  `in` (or NULL): every output row m is scaled by inv_m before
 * rounding, x being x' (the x rows of every problem).  `out` (or NULL; one problem only):
 * instead of writing y, h[m][n] += bf16(y[m][n]) (the bits a bf16 y added to h in fp32
 * gives), then x'[m][n] = bf16(h * weight[n]) and the per-tile sums of squares of the new
 * h for the next RMSNorm; the problem's y may be NULL.  x, y, h, x' and ssq must not
 * overlap.  M 1..32, K % 256 == 0; workspace of imq_qmv_norm_workspace bytes.  Same bits on
 * every call.  Replaces the projections of the reference's decode step together with the
 * RMSNorm before them and the residual add after them, ironmule/dense_plan.py:348-361.
 */
IMQ_API int32_t imq_qmv_norm(const imq_problem* problems, int32_t count, int32_t M,
                             int32_t group_size, int32_t bits, const imq_norm_in* in,
                             const imq_residual_out* out, float* workspace,
                             size_t workspace_bytes, void* stream);

/* K-ranges (output planes) imq_qmv_norm_planes splits these problems into at M rows; 0 if
 * the call would be refused. */
IMQ_API int32_t imq_qmv_norm_splits(const imq_problem* problems, int32_t count, int32_t M);

/*
 * imq_qmv_norm's input-norm form without the in-launch reduction of the K-ranges: each range
 * writes its fp32 partial product (row-scaled by inv_m when `in` is given) as an output
 * plane, and the reader of the result adds the planes in order (plane 0 first) and rounds:
 *   problem i, plane s, row m, column n at planes[i * pstride + (s * M + m) * N_i + n].
 * *splits receives the plane count (imq_qmv_norm_splits); pstride >= splits * M * max N_i.
 * The problems' y are not written (may be NULL).  Same limits as imq_qmv_norm; no workspace.
 * Replaces the same reference calls as imq_qmv_norm (the q/k/v projections of the decode
 * step, ironmule/dense_plan.py:348-353), for a reader that adds the planes itself
 * (imq_attention_fused_planes, ironmule_decode.h).  With x in the tile layout (every
 * problem's ldx == IMQ_LD_TILED, at most three problems of one K <= 4096) each problem is
 * one plane from bands of 32 weight rows over the whole K (*splits = 1).
 */
IMQ_API int32_t imq_qmv_norm_planes(const imq_problem* problems, int32_t count, int32_t M,
                                    int32_t group_size, int32_t bits, const imq_norm_in* in,
                                    float* planes, int64_t pstride, int32_t* splits, void* stream);

/*
 * imq_qmv_norm's residual epilogue (`out`) as a launch of its own, for one projection of N
 * columns computed as K-range planes by imq_qmv_norm_planes: y[m][n] = the nplanes planes
 * at planes[(s * M + m) * N + n] added in plane order from zero, then h += bf16(y),
 * x' = bf16(h * weight) and the per-tile sums of squares of the new h, with the bits of
 * imq_qmv_norm with that `out` over the same problem.  1 <= nplanes <= 16, 1 <= M <= 32; the
 * planes must not overlap h, x' or ssq.  The projection's launch then ends after its K-ranges
 * (no split counter or reload), and the epilogue runs on every CU instead of one workgroup
 * per 64-column tile.  Replaces the residual adds of the reference's decode step and the
 * RMSNorm after each, ironmule/dense_plan.py:348, 357-360.
 */
IMQ_API int32_t imq_residual_planes(const float* planes, int32_t nplanes, int32_t M, int32_t N,
                                    const imq_residual_out* out, void* stream);

/*
 * The 32-row tile layout of a bf16 activation of M <= 32 rows and K columns (K a multiple of
 * 64), selected by the row stride IMQ_LD_TILED where an entry point accepts it: element
 * (m, k) at element offset
 *   ((((k / 64) * 4 + (k % 32) / 8) * 2 + (k % 64) / 32) * 32 + m) * 8 + k % 8,
 * a buffer of 32 * K elements whatever M (rows m >= M are neither read nor written).  Each
 * 64-column group is 4 KB in which the 16 bytes an MFMA lane (m, half) reads for one k-step
 * lie next to those of the other 63 lanes, so the batched kernels read the activation as
 * contiguous 1 KB pieces instead of 32 rows x 32 bytes.  No reference counterpart: the
 * layout in which the decode step's launches hand activations to one another.
 */
#define IMQ_LD_TILED 0

/*
 * imq_qmv_norm's residual form for one projection (no input norm) over bands of 32 weight
 * rows and the whole K, a workgroup per band: y = x W^T is never written and the K-ranges
 * never leave the workgroup (no partials, planes or epilogue launch); then h += bf16(y),
 * x' = bf16(h * weight) and, per band of 32 columns, each row's sum of squares of the new
 * h: ssq[m * ld + t], t < ceil(N / 32) (`ld` a multiple of 4, at least that).  x as rows
 * (ldx >= K, a multiple of 8) or in the tile layout (ldx == IMQ_LD_TILED); M 1..32,
 * K a multiple of 256 and at most 9728.  Same bits on every call.  Replaces the o and down
 * projections of the reference's decode step with the residual add after each and the
 * RMSNorm after that, ironmule/dense_plan.py:357-361.
 */
IMQ_API int32_t imq_qmv_residual_bands(const imq_problem* problem, int32_t M, int32_t group_size,
                                       int32_t bits, const imq_residual_out* out, void* stream);

/* Bytes of workspace imq_qmv_gate_up_silu_norm uses at these shapes (0: none): when the
 * launch's 32-row tiles make more than one round over the CUs, the tiles of the last,
 * partial round are cut into K-parts that occupy the CUs the whole tiles leave free. */
IMQ_API size_t imq_qmv_gate_up_silu_norm_workspace(int32_t M, int32_t N, int32_t K);

/*
 * imq_qmv_gate_up_silu on x' rows with the input RMSNorm folded in (`in` non-NULL):
 *   act[m][n] = bf16(silu(g) * u),  g = bf16(inv_m * sum_k x'[m][k] W_gate[n][k]),
 *                                   u = bf16(inv_m * sum_k x'[m][k] W_up[n][k]).
 * Same shapes and limits as imq_qmv_gate_up_silu, except that any M from 1 to 32 is taken
 * (the decode step folds its norms from 3 rows).  K of 4, 8, 10 or 12 times 256 runs one
 * workgroup per CU over bands of 8-row units of both weights and the whole K (no
 * workspace; x and act may then be in the tile layout, ldx / ld_act == IMQ_LD_TILED).
 * Otherwise, with a workspace of imq_qmv_gate_up_silu_norm_workspace bytes (zero-filled
 * before its first use and left ready by every call; calls sharing one must not overlap)
 * the last round's 32-row tiles are cut into K-parts whose sums are added in part order;
 * with none (NULL, 0 bytes) every tile is whole.  Replaces the post-attention RMSNorm, the
 * fused gate/up launch and the SwiGLU, ironmule/dense_plan.py:359-360 and
 * ironmule/fast.py:186-215.
 */
IMQ_API int32_t imq_qmv_gate_up_silu_norm(const uint32_t* w_gate, const uint16_t* s_gate,
                const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up,
                const uint16_t* b_up, const uint16_t* x, int64_t ldx, uint16_t* act,
                int64_t ld_act, int32_t M, int32_t N, int32_t K, int32_t group_size,
                int32_t bits, const imq_norm_in* in, float* workspace, size_t workspace_bytes,
                void* stream);

/*
 * The same product for `count` separate activation vectors xs[i] (each (1, K)) and
 * separate outputs ys[i] (each (1, N)), one weight sweep for all of them.
 *
 * Replaces:
 *   ironmule/qmv_shared.py:169-181       run_shared(w, scales, biases, vectors, N)  (K = 3840)
 *   ironmule/qmv_fast_shared.py:161-172  run_fast(w, scales, biases, vectors, N, K)
 * `xs` and `ys` are host arrays of `count` device pointers (1 <= count <= 32).
 */
IMQ_API int32_t imq_qmv_multi(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      const uint16_t* const* xs, void* const* ys, int32_t count, int32_t N,
                      int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype,
                      void* stream);

/*
 * imq_qmv for `count` (1..IMQ_MAX_PROBLEMS) weights in one launch, every one with the
 * same M, group size, bits and output dtype; each weight is read once for its M rows.
 * Projections that read the same activation (q/k/v, gate/up) take the same x pointer.
 *
 * Replaces the reference's fused projection groups, ironmule/fast.py:186-215
 * (fuse_projections: q/k/v and gate/up concatenated into one quantised linear so one
 * launch serves them); here the weights stay separate buffers and the launch is shared.
 */
IMQ_API int32_t imq_qmv_grouped(const imq_problem* problems, int32_t count, int32_t M,
                                int32_t group_size, int32_t bits, int32_t y_dtype,
                                void* stream);

/* Bytes of workspace imq_qmv_grouped_ws can use for these problems at M rows: with it the
 * groups of weights with few rows (for a given K) are split over more workgroups (fp32
 * partials, which the last workgroup of each tile adds in a fixed order, in the same
 * launch).  0 when no split helps (M < 3 or enough rows). */
IMQ_API size_t imq_qmv_grouped_workspace(const imq_problem* problems, int32_t count, int32_t M);

/* imq_qmv_grouped with a caller-provided workspace of workspace_bytes (16-byte aligned;
 * may be 0 bytes, then no split).  The workspace must be zero-filled before its first
 * use; every call leaves it ready for the next (its tile counters back at zero), so one
 * workspace serves any number of calls.  Same results as imq_qmv_grouped up to the fp32
 * summation order of the splits, and the same bits on every call; calls that share a
 * workspace must not overlap.
 * Replaces the same reference calls as imq_qmv_grouped, and imq_qmv at M >= 3 (the
 * shared-weight form, ironmule/cuda_native.py:155-168 for M <= 8, up to 32 here). */
IMQ_API int32_t imq_qmv_grouped_ws(const imq_problem* problems, int32_t count, int32_t M,
                                   int32_t group_size, int32_t bits, int32_t y_dtype,
                                   float* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the library's static split scratch (one per device, held until the process
 * ends), the largest split workspace imq_qmv_grouped_noalloc serves. */
#define IMQ_NOALLOC_SCRATCH_BYTES (8u << 20)

/*
 * imq_qmv_grouped_ws without a caller workspace and without any allocation: the split
 * partials and counters live in the library's own static device scratch (a per-device
 * array of IMQ_NOALLOC_SCRATCH_BYTES), so the call performs no hipMalloc, hipFree or other
 * allocation and can be made where allocating is not allowed.  Same plan, hence the same
 * bits, as imq_qmv_grouped_ws given imq_qmv_grouped_workspace bytes.  A call whose split
 * workspace would exceed the scratch returns IMQ_EUNSUPPORTED.  When the call splits, a
 * small fill kernel clears the scratch's counters first (two launches on `stream`).
 * Every call on one device shares that device's scratch: calls that overlap on a device
 * (different streams, or threads) race and must be serialised by the caller.
 * No counterpart in the reference: this entry point is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 */
IMQ_API int32_t imq_qmv_grouped_noalloc(const imq_problem* problems, int32_t count, int32_t M,
                                        int32_t group_size, int32_t bits, int32_t y_dtype,
                                        void* stream);

/* MoE gather: for each of `pairs` (token, expert) pairs p, the one-row product
 *   y[p] = x[p / rows_per_x] W[idx[p]]^T
 * where w, scales and biases hold `experts` stacked weights ((E, N, K/8) words and
 * (E, N, K/64) bf16) and idx (pairs uint32, device memory) names each pair's expert.
 * rows_per_x = 1 gives every pair its own activation row (a down projection); a larger
 * value lets that many consecutive pairs share one row (gate/up: one token's row for all
 * of its experts).  Each pair's row equals imq_qmv on that expert's weights, bit for bit.
 * An index outside [0, experts) yields a row of zeros.  N * K / 64 must be even.
 * Replaces the reference's gather kernel and routing, ironmule/cuda_native.py:130-144
 * (ironmule_native_gather4) and 182-218 (_gather_qmv, gather_matmul). */
IMQ_API int32_t imq_gather_qmv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                               int32_t experts, const uint16_t* x, int64_t ldx, int32_t rows_per_x,
                               const uint32_t* idx, int32_t pairs, void* y, int64_t ldy, int32_t N,
                               int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype,
                               void* stream);

/*
 * out[n][k] = scales[n][k/64] * q[n][k] + biases[n][k/64] as fp32 (bit-exact:
 * scale*q is exact in fp32, so only the add rounds), or that fp32 value rounded
 * to bf16 / fp16 (nearest even) per out_dtype.  out is (N, K) contiguous.
 *
 * Replaces mx.dequantize on the path:
 *   ironmule/cuda_native.py:177-179      prefill: dequantise (fp16) then GEMM
 *   ironmule/cuda_native.py:265-266      probe reference: dequantise with fp32 scales
 *   ironmule/numeric_plans.py:462-464    the `dequantize` plan's fp32 weights
 */
IMQ_API int32_t imq_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    void* out, int32_t out_dtype, int32_t N, int32_t K, int32_t group_size,
                    int32_t bits, void* stream);

/* Copies the calling thread's last error message (NUL-terminated, truncated to
 * len) and returns the last error code (IMQ_OK if none). */
IMQ_API int32_t imq_last_error(char* buf, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* IRONMULE_QMV_H */
