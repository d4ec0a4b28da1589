/*
 * ironmule_step.h — C ABI of the persistent decode-step engine for MI355X (gfx950), in
 * libironmule_qmv.so.
 *
 * A "program" is a list of stages run by ONE persistent kernel launch: every stage is a
 * set of independent tasks (tiles of a 4-bit qmv, or (request, KV head, key range)
 * pieces of decode attention), and a stage may wait for every task of an earlier stage.
 * Workgroups take tasks in a fixed round-robin order; a task issues its weight loads,
 * then waits for its input stage, so the weight stream of later stages keeps HBM busy
 * while the activations of earlier ones are still being produced.  This replaces the
 * per-kernel launches of a decode step (the reference issues one kernel per projection
 * and per attention piece: ironmule/dense_plan.py:337-363, cuda_native.py:155-168).
 *
 * Contract:
 *   * Creation validates shapes, plans the tasks and allocates the program's device
 *     tables, activation buffers and counters (hipMalloc); launches allocate nothing.
 *   * A launch enqueues two kernels on `stream` (a counter reset, then the persistent
 *     kernel) and can be captured in a HIP graph.  Launches of one program must not
 *     overlap, and no other kernel may run on the device while one runs (the persistent
 *     kernel assumes its workgroups are co-resident).
 *   * Every wait inside the kernel is bounded: if a stage does not complete in time (it
 *     cannot, unless the co-residency assumption is broken) the kernel stops and
 *     imq_program_status() reports it.
 *   * A qmv program's results are bit-identical to the per-kernel path (imq_qmv /
 *     imq_qmv_grouped) on the same inputs: every stage uses the same arithmetic in the
 *     same order.  A decode program folds its RMSNorms into the projections (below); its
 *     persistent and staged launches give each other's bits.
 *   * Return codes are the IMQ_* values of ironmule_qmv.h, with imq_last_error().
 */
#ifndef IRONMULE_STEP_H
#define IRONMULE_STEP_H

#include <stddef.h>
#include <stdint.h>

#include "ironmule_qmv.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct imq_program imq_program; /* opaque */

/* One 4-bit group-64 weight: packed words (N, K/8), bf16 scales and biases (N, K/64). */
typedef struct {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases;
} imq_qweight;

/* The tensors of one Qwen3-style decoder layer. */
typedef struct {
  imq_qweight q, k, v, o, gate, up, down;
  const uint16_t* input_norm; /* bf16 (hidden) */
  const uint16_t* post_norm;  /* bf16 (hidden) */
  const uint16_t* q_norm;     /* bf16 (128) */
  const uint16_t* k_norm;     /* bf16 (128) */
  uint16_t* k_pool;           /* bf16 (num_slots, kv_heads, capacity, 128) */
  uint16_t* v_pool;
} imq_step_layer;

/* A decode step of a Qwen3-style decoder at batch 1: for the request's token already
 * embedded in h (imq_embed),
 *   per layer: x = rms_norm(h) ; q,k,v = x W^T ; q,k = rope(rms_norm_head(q, k)) at
 *              positions[0] ; KV[slot][pos] = k, v ; o = attention over keys 0..pos ;
 *              h += bf16(o Wo^T) ; x = rms_norm(h) ;
 *              h += bf16(bf16(silu(bf16(x Wg^T)) * bf16(x Wu^T)) Wd^T)
 *   logits = rms_norm(h) E^T (fp32)
 * with the per-kernel path's rounding points (ironmule_decode.h) except that every
 * RMSNorm but the first layer's input norm is folded into the projections around it: the
 * o and down stages also write x' = bf16(h * w_next) and one sum of squares of the new h
 * per tile, and the next stage computes inv * (x' W^T) with inv = 1 / rms(h) from those
 * sums, rounding x before the scaling instead of after it (imq_qmv_norm's arithmetic at one
 * row; logits within about 5e-4 of the unfolded step's, relative to their maximum).  A request
 * whose slot is outside [0, num_slots) or whose position is outside [0, capacity) gets
 * no KV write and zeros from attention.
 * Replaces DensePlan.forward's decode step (ironmule/dense_plan.py:337-363;
 * ironmule/dense_cpu.py:188-220) for one request. */
typedef struct {
  int32_t layers, batch, hidden, heads, kv_heads, intermediate, vocab;
  int32_t capacity, num_slots, max_len;
  float eps, theta;
  const imq_step_layer* layer; /* `layers` entries; read during creation only */
  const uint16_t* final_norm;  /* bf16 (hidden) */
  imq_qweight head;            /* (vocab, hidden) */
  const int32_t* positions;    /* device, `batch` entries, read at every launch */
  const int32_t* slots;        /* device, `batch` entries, read at every launch */
  float* h;                    /* device (batch, hidden) fp32 residual stream, updated */
  float* logits;               /* device (batch, vocab) fp32, written */
} imq_step_desc;

IMQ_API int32_t imq_decode_program_create(const imq_step_desc* desc, imq_program** out);

/* A chain of 4-bit qmv stages at one activation row (M = 1): stage i computes
 * y_p = x_p W_p^T (bf16) for its problems (1..3, the imq_problem fields x, y, N, K and
 * the weights; M, ldx, ldy ignored), and when wait_previous is set it starts only after
 * stage i-1 has finished (so it may read stage i-1's outputs).  Each output element is
 * the same value imq_qmv computes.
 * Replaces a sequence of qmv launches (ironmule/qmv_k3840.py:299-310; the grouped form
 * of ironmule/fast.py:186-215). */
typedef struct {
  int32_t count;
  int32_t wait_previous;
  imq_problem problems[3];
} imq_qmv_stage;

IMQ_API int32_t imq_qmv_program_create(const imq_qmv_stage* stages, int32_t count,
                                       imq_program** out);

/* Enqueues one run of the program on `stream`: every stage in one persistent launch. */
IMQ_API int32_t imq_program_launch(imq_program* program, void* stream);

/* Enqueues one run of the program on `stream` as one launch per stage (each workgroup
 * runs one task, the stream order replaces the waits); the same results as
 * imq_program_launch, bit for bit. */
IMQ_API int32_t imq_program_launch_staged(imq_program* program, void* stream);

/* Waits for the device, then sets *failed to 1 if a run since the last call stopped on
 * a bounded wait (0 otherwise) and clears the flag. */
IMQ_API int32_t imq_program_status(imq_program* program, int32_t* failed);

/* Tasks, stages, persistent workgroups and LDS bytes per workgroup of the program. */
IMQ_API int32_t imq_program_info(const imq_program* program, int32_t* tasks, int32_t* stages,
                                 int32_t* workgroups, int32_t* lds_bytes);

IMQ_API void imq_program_destroy(imq_program* program);


/* ------------------------------------------------------------------ streaming engine
 *
 * A chain of one-row 4-bit qmv stages (imq_qmv_stage, as for imq_qmv_program_create)
 * run by ONE persistent launch that streams the weights of every stage; each wavefront
 * keeps its next tile's loads in flight while it computes the current one.
 *   * With no wait_previous anywhere the stages are independent: their distinct x rows
 *     (at most 8, 64 KiB staged) are read once per workgroup at the start and the
 *     wavefronts stream from the first stage to the last with no barrier or wait, each
 *     taking every V-th run of consecutive tiles (V wavefronts; 16 or more tiles per run
 *     when the program has at least 16 tiles per wavefront).
 *   * With waits, each wavefront takes every V-th tile of a stage.
 *     Every workgroup enters the stages in order, issuing its weight loads
 *     for a stage before waiting for that stage's input; the grid is then limited to the
 *     workgroups the device keeps resident at once, no other kernel may run on the device
 *     during the launch, and every wait is bounded (imq_stream_status reports a stall).
 * Each output element is the value imq_qmv computes for the same inputs, bit for bit.
 * `workgroups` <= 0 picks the resident maximum.  Creation allocates the program's device
 * tables (hipMalloc); a launch allocates nothing and can be captured in a HIP graph.
 * Replaces a sequence of qmv launches (ironmule/qmv_k3840.py:299-310, the grouped form
 * of ironmule/fast.py:186-215, and the chained weights of the reference's bandwidth
 * measurement, ironmule/hw.py:441-473). */
typedef struct imq_stream imq_stream; /* opaque */

IMQ_API int32_t imq_stream_create(const imq_qmv_stage* stages, int32_t count, int32_t workgroups,
                                  imq_stream** out);

/* Enqueues one run on `stream` (for a chained program: a counter reset, then the kernel). */
IMQ_API int32_t imq_stream_launch(imq_stream* program, void* stream);

/* Waits for the device; *failed = 1 if a run since the last call stopped on a bounded
 * wait (then clears the flag). */
IMQ_API int32_t imq_stream_status(imq_stream* program, int32_t* failed);

/* A diagnostic with no counterpart in the reference: later launches of a chained program
 * record, per (stage s, wavefront v) at buffer[(s * V + v) * 4 ..], four s_memrealtime
 * stamps (a 100 MHz clock): the stage's start (after the workgroup signalled the previous
 * stage), its input ready (the wait for the previous stage done), its x staged in LDS and
 * its last tile done.  V = workgroups * 12 (imq_stream_info); `words` >= stages * V * 4.  A
 * NULL buffer stops the recording.  IMQ_EUNSUPPORTED for a program without waits. */
IMQ_API int32_t imq_stream_trace(imq_stream* program, uint64_t* buffer, int64_t words);

/* Tiles, stages, workgroups, LDS bytes per workgroup, and 1 if the stages are chained. */
IMQ_API int32_t imq_stream_info(const imq_stream* program, int32_t* tiles, int32_t* stages,
                                int32_t* workgroups, int32_t* lds_bytes, int32_t* chained);

IMQ_API void imq_stream_destroy(imq_stream* program);

#ifdef __cplusplus
}
#endif

#endif /* IRONMULE_STEP_H */
