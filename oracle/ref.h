/* oracle/ref.h - CPU oracle for the decode hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load or call this code, and only as the checker (or the timed CPU
 * baseline), never as part of the product path. The product library
 * (surge_amd/libsurge_amd.so) does not link it.
 *
 * The functions restate the reference's scalar CPU reference
 * (reference src/ref.c) with its exact numerics: every reduction accumulates
 * in double in strictly increasing index order, transcendentals are libm's
 * double versions, and results are rounded to f32 where the reference rounds
 * them. Names and argument meanings follow the reference's declarations in
 * its surge.h:349-638 so tests read like the reference's own.
 */
#ifndef SURGE_ORACLE_REF_H
#define SURGE_ORACLE_REF_H

#include "../include/surge.h"

#ifdef __cplusplus
extern "C" {
#endif

float sg_ref_f16_to_f32(uint16_t h);                 /* ref.c:80-107 */
void sg_ref_rmsnorm(float *x, const float *w, uint32_t n, float eps);  /* ref.c:113-125 */
float sg_ref_sigmoid(float x);                       /* ref.c:127-134 */
float sg_ref_softplus(float x);                      /* ref.c:136-142 */
float sg_ref_delta_decay(float a_log, float a, float dt_bias);        /* ref.c:144-150 */
float sg_ref_delta_decay_neg_a(float neg_a, float a, float dt_bias);  /* ref.c:152-170 */
void sg_ref_silu(float *x, uint32_t n);              /* ref.c:172-175 */
void sg_ref_swiglu(float *gate, const float *up, uint32_t n);         /* ref.c:177-183 */
void sg_ref_gate_sigmoid(float *x, const float *gate, uint32_t n);    /* ref.c:185-188 */
void sg_ref_softmax(float *x, uint32_t n);           /* ref.c:190-235 */
void sg_ref_attn_combine(const float *m, const float *s, const float *acc,
                         uint32_t n_parts, uint32_t head_dim, float *out);  /* ref.c:265-373 */
void sg_ref_attn_decode(const float *q, const float *kc, const float *vc,
                        uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                        uint32_t seq, uint32_t q_stride, float scale, float *out); /* ref.c:541-546 */
void sg_ref_attn_decode_splitk(const float *q, const float *kc, const float *vc,
                               uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                               uint32_t seq, uint32_t q_stride, float scale,
                               uint32_t n_parts, float *out);  /* ref.c:549-555 */
/* The per-(head, split) partial triple the split-K combine consumes
 * (ref.c:416-455), exposed so GPU partials can be compared before combining.
 * m, s: [n_heads, n_parts]; acc: [n_heads, n_parts, head_dim]. */
void sg_ref_attn_partials(const float *q, const float *kc, const float *vc,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t seq, uint32_t q_stride, float scale,
                          uint32_t n_parts, float *m, float *s, float *acc);
void sg_ref_rope_partial(float *q, uint32_t head_dim, uint32_t rope_dim,
                         uint32_t pos, float theta);  /* ref.c:561-602 */
void sg_ref_rope(float *q, uint32_t head_dim, uint32_t pos, float theta); /* ref.c:604-606 */
void sg_ref_matvec_f32(const float *w, const float *x, float *y,
                       uint32_t rows, uint32_t cols);  /* ref.c:612-621 */
void sg_ref_matvec_bf16(const uint16_t *w, const float *x, float *y,
                        uint32_t rows, uint32_t cols); /* ref.c:623-632 */
void sg_ref_matvec_q8(const void *w, const float *x, float *y,
                      uint32_t rows, uint32_t cols);   /* ref.c:638-663 */
void sg_ref_conv1d_causal(float *x, const float *w, const float *state_in,
                          float *state_out, uint32_t channels, uint32_t ksize); /* ref.c:669-706 */
void sg_ref_delta_step(float *S, const float *q, const float *k, const float *v,
                       float beta, float decay, float *out,
                       uint32_t dk, uint32_t dv);      /* ref.c:708-739 */

/* Whole-model forward (ref.c:862-1386). */
typedef struct sg_ref_state sg_ref_state;
sg_err sg_ref_state_new(const sg_model *m, uint32_t max_ctx, sg_ref_state **out);
void sg_ref_state_free(sg_ref_state *st);
void sg_ref_state_reset(sg_ref_state *st);
sg_err sg_ref_forward(sg_ref_state *st, const sg_model *m, int32_t token,
                      uint32_t pos, const float **logits);
/* Oracle-only switch (no reference counterpart): store K/V rounded through
 * f16 round-to-nearest-even, as the GPU's f16 KV cache does, so a
 * GPU-vs-oracle comparison can separate the KV storage rounding from
 * everything else. Off by default (the reference keeps f32 K/V). */
void sg_ref_state_set_kv_f16(sg_ref_state *st, bool on);
/* Test input: the seeded state sg_gpu_state_fill_synthetic writes, in this
 * state's layouts; the next forward is at position n. */
sg_err sg_ref_state_fill_synthetic(sg_ref_state *st, uint32_t n, uint32_t seed);

uint16_t sg_ref_f32_to_f16(float f);                 /* kv.c:152-190 */
uint32_t sg_ref_argmax_f32(const float *v, uint32_t n);  /* greedy.c:17-27 */

/* Sets the OpenMP thread count for the row-parallel matvecs (rows are
 * independent, so any count gives bit-identical results); returns the count
 * in effect. 1 when built without OpenMP. */
int sg_ref_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
