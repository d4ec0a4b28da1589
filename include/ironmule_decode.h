/*
 * ironmule_decode.h — C ABI of the decode-step kernels that sit between the 4-bit qmv
 * launches of a Qwen3-style decoder on MI355X (gfx950), in libironmule_qmv.so.
 *
 * One decode step of B requests (each its own KV slot and position), as the reference
 * composes it (ironmule/dense_plan.py:337-363, ironmule/dense_cpu.py:188-220):
 *   h = embed(tokens)
 *   per layer: x = rms_norm(h) ; q,k,v = qmv(x) ; q,k = rope(rms_norm_head(q,k)) ;
 *              KV[slot][pos] = k,v ; o = attention(q, KV[slot][:pos+1]) ;
 *              h += qmv_o(o) ; x = rms_norm(h) ; h += qmv_down(silu(qmv_gate(x)) * qmv_up(x))
 *   logits = qmv_head(rms_norm(h))
 * The projections are imq_qmv / imq_qmv_grouped (ironmule_qmv.h); these entry points are
 * the rest.
 *
 * Contract (as for ironmule_qmv.h): device pointers allocated by the caller, work queued
 * on `stream`, no allocation or synchronisation per call, int32 return codes (IMQ_*
 * values of ironmule_qmv.h) with imq_last_error() for the message.
 *
 * Layouts:
 *   h         fp32 (B, dim): the residual stream
 *   bf16      activations (B, dim) and heads (B, H, 128)
 *   KV pool   bf16 (slots, kv_heads, capacity, 128) per layer, the reference's pool layout
 *             (dense_plan.py:297-301, rows = (slot * kv_heads + head) * capacity + position)
 */
#ifndef IRONMULE_DECODE_H
#define IRONMULE_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "ironmule_qmv.h"

#ifdef __cplusplus
extern "C" {
#endif

#define IMQ_HEAD_DIM 128

/* h[b][:] = dequantised embedding row tokens[b] (4-bit, group 64, bf16 scales/biases, the
 * qmv weight format), as fp32.  Tokens outside [0, vocab) are refused by the kernel:
 * their rows are written as NaN.
 * Replaces trunk.embed_tokens(tokens) (ironmule/dense_plan.py:343; dense_cpu.py:200). */
IMQ_API int32_t imq_embed(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                          const int32_t* tokens, float* h, int32_t B, int32_t vocab, int32_t dim,
                          void* stream);

/* The first half of an RMSNorm folded into the projection that follows it: if delta is
 * non-NULL, h += delta (bf16) first; then out = bf16(h * weight) (not normalised) and
 * ssq[b * ld] = sum of h[b][:]^2, the one partial sum per row that imq_qmv_norm or
 * imq_qmv_gate_up_silu_norm (ironmule_qmv.h, imq_norm_in with tiles = 1) turns into the row's
 * 1/rms.  ssq 16-byte aligned, ld a multiple of 4; dim <= 8192.
 * Replaces the input RMSNorm of the first layer, ironmule/dense_plan.py:348. */
IMQ_API int32_t imq_rmsnorm_prescale(float* h, const uint16_t* delta, const uint16_t* weight,
                                     uint16_t* out, float* ssq, int32_t ld, int32_t B, int32_t dim,
                                     void* stream);

/* If delta is non-NULL, h += delta (bf16) first; then out = bf16(h * rsqrt(mean(h^2) + eps)
 * * weight), per row of dim values (dim <= 8192).
 * Replaces mx.fast.rms_norm(h, weight, eps) and the residual adds `h = h + ...`
 * (ironmule/dense_plan.py:348, 358-359, 362). */
IMQ_API int32_t imq_add_rmsnorm(float* h, const uint16_t* delta, const uint16_t* weight,
                                uint16_t* out, int32_t B, int32_t dim, float eps, void* stream);

/* Per request b and head: q heads and k heads get the per-head RMSNorm (q_norm / k_norm
 * weights, rounded to bf16 as the reference's module output) and the non-interleaved
 * rotary embedding at positions[b] with base `theta`; q goes to q_out (B, Hq, 128); k and
 * the untouched v go to the KV pools (num_slots slots of `capacity` positions) at
 * (slots[b], head, positions[b]).  A request whose position is not in [0, capacity) or
 * whose slot is not in [0, num_slots) is refused: nothing is written for it.
 * Replaces q_norm/k_norm + _rope + the KV write (ironmule/dense_plan.py:349-356, 365-371). */
IMQ_API int32_t imq_qk_norm_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* q_norm, const uint16_t* k_norm,
                                 const int32_t* positions, const int32_t* slots, uint16_t* q_out,
                                 uint16_t* k_pool, uint16_t* v_pool, int32_t B, int32_t Hq,
                                 int32_t Hkv, int32_t capacity, int32_t num_slots, float theta,
                                 float eps, void* stream);

/* Bytes of fp32 workspace imq_attention_decode needs for B requests, Hq query heads and
 * keys up to max_len (at most one partial result per 64-key chunk). */
IMQ_API size_t imq_attention_workspace(int32_t B, int32_t Hq, int32_t max_len);

/* out[b][h] = softmax(scale * q[b][h] . K[slot][h/G][:len]) V[slot][h/G][:len] with
 * slot = slots[b], len = lengths[b] (clamped to max_len and capacity), G = Hq / Hkv <= 8
 * query heads per KV head (grouped-query attention).  A request with len <= 0 or a slot
 * outside [0, num_slots) gets zeros.  The keys of each (request, KV head) are split over
 * several workgroups (whole 64-key chunks each, enough splits to fill the GPU); a second
 * launch merges the splits in split order, so the result does not depend on scheduling.
 * Calls that share `workspace` must not overlap.
 * Replaces fa2 (ironmule/dense_plan.py:258-274): the FA2_PARTIAL / FA2_COMBINE pair. */
IMQ_API int32_t imq_attention_decode(const uint16_t* q, const uint16_t* k_pool,
                                     const uint16_t* v_pool, const int32_t* lengths,
                                     const int32_t* slots, uint16_t* out, int32_t B, int32_t Hq,
                                     int32_t Hkv, int32_t capacity, int32_t num_slots,
                                     int32_t max_len, float scale, float* workspace,
                                     void* stream);

/* The attention of one decode step fused into one launch, as the decode programs run it:
 * per-head RMSNorm (q_norm, k_norm, eps) and rotary embedding (theta, at positions[b])
 * of q (B, Hq, 128) and k (B, Hkv, 128); this step's k and v written into the pools at
 * row positions[b] of slot slots[b]; then out[b][h] = softmax(q . K / sqrt(128)) V over
 * rows 0 .. positions[b] of the slot (clamped to max_len and capacity), split over 64-key
 * chunks with the split plan of imq_attention_decode and merged in split order by the
 * last split of each (request, KV head); from 64 (request, KV head) pairs a workgroup of
 * 12 wavefronts per task, split so that about 256 tasks run (never more splits than that
 * plan; none from 256 pairs).  The KV pools get the same bits as
 * imq_qk_norm_rope followed by imq_attention_decode with lengths = positions + 1 for every
 * valid request, and the output agrees with theirs to the attention's oracle bar (the
 * scores and P.V run on MFMA, in another summation order); a request with
 * its slot outside [0, num_slots) or its position outside [0, capacity) is invalid: its
 * output is zeros and it writes nothing (as imq_attention_decode with length 0; given the
 * length positions + 1 past the capacity that entry would attend over the stored rows of a
 * valid slot).  `workspace`: at least
 * imq_attention_workspace(B, Hq, max_len) bytes; `counters`: B * Hkv uint32, zero before
 * the first call and left at zero by every call (one set per stream).  Replaces the
 * q_norm, k_norm, rope, KV write and attention steps of the decode composition
 * (ironmule/dense_cpu.py:201-220). */
IMQ_API int32_t imq_attention_fused(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    const uint16_t* q_norm, const uint16_t* k_norm,
                                    const int32_t* positions, const int32_t* slots,
                                    uint16_t* k_pool, uint16_t* v_pool, uint16_t* out, int32_t B,
                                    int32_t Hq, int32_t Hkv, int32_t capacity, int32_t num_slots,
                                    int32_t max_len, float theta, float eps, float* workspace,
                                    uint32_t* counters, void* stream);

/* imq_attention_fused with q, k and v given as the fp32 output planes of a split projection
 * (imq_qmv_norm_planes over the q, k and v weights, ironmule_qmv.h) instead of bf16 rows:
 * each q/k/v value is the sum of its `nplanes` planes (1..4) in plane order, rounded to bf16,
 * problem i (0 q, 1 k, 2 v), plane s, request b at planes[i * pstride + (s * B + b) * N_i]
 * with N_i = Hq * 128 or Hkv * 128.  out: rows of Hq * 128 (ld_out = Hq * 128) or, for at most
 * 32 requests, the 32-row tile layout (ld_out = IMQ_LD_TILED, ironmule_qmv.h) that the o
 * projection reads in contiguous pieces.  Otherwise as imq_attention_fused.  Replaces the
 * same reference steps, with the q/k/v projections' final reduction folded in
 * (ironmule/dense_plan.py:348-357). */
IMQ_API int32_t imq_attention_fused_planes(const float* planes, int64_t pstride, int32_t nplanes,
                                           const uint16_t* q_norm, const uint16_t* k_norm,
                                           const int32_t* positions, const int32_t* slots,
                                           uint16_t* k_pool, uint16_t* v_pool, uint16_t* out,
                                           int64_t ld_out, int32_t B, int32_t Hq, int32_t Hkv,
                                           int32_t capacity, int32_t num_slots, int32_t max_len,
                                           float theta, float eps, float* workspace, uint32_t* counters,
                                           void* stream);

/* out = bf16(silu(gate) * up), silu(g) = g / (1 + exp(-g)), n elements.
 * Replaces swiglu(gate, up) (ironmule/dense_plan.py:360; nn.silu in dense_cpu.py:216). */
IMQ_API int32_t imq_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                             void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IRONMULE_DECODE_H */
