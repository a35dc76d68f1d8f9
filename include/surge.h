/* surge.h - the public C ABI of the MI355X decode engine.
 *
 * This header keeps the reference engine's C interface for the batch-1
 * decode hot path (reference: surge.h), so a caller written against the
 * reference links against this library unchanged. Every declaration below
 * cites the reference declaration it replaces as `surge.h:LINE` (reference
 * file, not this one). Types that cross the boundary (sg_err, sg_tensor,
 * sg_cfg, sg_layer_w, sg_model) keep the reference's field order and widths
 * exactly, so one sg_model value can be handed to this library, to the
 * reference's CPU oracle and to this repository's CPU oracle alike.
 *
 * Semantic differences from the reference, all forced by discrete memory
 * (the reference targets a unified-memory GPU):
 *   - sg_gpu_wrap COPIES the caller's bytes into HBM (the reference wraps
 *     them with no copy). The caller's memory need not outlive the handle.
 *   - sg_gpu_alloc's *host_out is a HOST MIRROR of the device buffer, not the
 *     same memory. Every synchronous one-shot entry point (sg_gpu_run_*)
 *     uploads each argument buffer's mirror before launching and downloads
 *     every buffer the kernel writes into its mirror after the launch has
 *     finished, so "write host, call, read host" works as in the reference.
 *   - Buffers made by sg_gpu_wrap_device have no mirror: they wrap memory
 *     that is already on the device (e.g. a torch tensor) and are never
 *     copied. This is an addition for callers that keep data in HBM.
 *   - sg_gpu_forward's logits are copied device-to-host once per token.
 */
#ifndef SURGE_H
#define SURGE_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error convention (surge.h:7-11): msg == NULL means success. Messages are
 * static strings or a static format buffer, so they are not thread-safe. */
typedef struct { const char *msg; } sg_err;
#define SG_OK ((sg_err){0})
static inline bool sg_failed(sg_err e) { return e.msg != NULL; }

/* ---------------------------------------------------------------------
 * GGUF v3 reader (surge.h:13-46)
 * --------------------------------------------------------------------- */
typedef enum { SG_GGUF_U8 = 0, SG_GGUF_I8, SG_GGUF_U16, SG_GGUF_I16, SG_GGUF_U32,
  SG_GGUF_I32, SG_GGUF_F32, SG_GGUF_BOOL, SG_GGUF_STR, SG_GGUF_ARR, SG_GGUF_U64,
  SG_GGUF_I64, SG_GGUF_F64 } sg_gguf_kv_type;
typedef enum { SG_T_F32 = 0, SG_T_F16 = 1, SG_T_Q8_0 = 8, SG_T_BF16 = 30 } sg_tensor_type;
typedef struct { const char *name; sg_tensor_type type; uint32_t n_dims;
  uint64_t dims[4]; const void *data; uint64_t nbytes; } sg_tensor;
typedef struct sg_gguf sg_gguf;

sg_err sg_gguf_open(const char *path, sg_gguf **out);              /* surge.h:22 */
void sg_gguf_close(sg_gguf *g);                                      /* surge.h:23 */
bool sg_gguf_get_u32(const sg_gguf *g, const char *key, uint32_t *out);   /* surge.h:25 */
bool sg_gguf_get_f32(const sg_gguf *g, const char *key, float *out);      /* surge.h:26 */
bool sg_gguf_get_str(const sg_gguf *g, const char *key, const char **out);/* surge.h:27 */
/* Array metadata (surge.h:28-35): element type, raw data pointer (for
 * non-string arrays) and element count. */
bool sg_gguf_get_arr(const sg_gguf *g, const char *key, sg_gguf_kv_type *elem_type,
                     const void **data, uint64_t *count);
uint32_t sg_gguf_version(const sg_gguf *g);                          /* surge.h:41 */
uint64_t sg_gguf_kv_count(const sg_gguf *g);                         /* surge.h:42 */
const sg_tensor *sg_gguf_tensor(const sg_gguf *g, const char *name); /* surge.h:44 */
uint64_t sg_gguf_tensor_count(const sg_gguf *g);                     /* surge.h:45 */
const sg_tensor *sg_gguf_tensor_at(const sg_gguf *g, uint64_t i);    /* surge.h:46 */

/* ---------------------------------------------------------------------
 * Model description (surge.h:115-347)
 * --------------------------------------------------------------------- */

/* Model config (surge.h:115-151). key_dim = n_k_heads*head_k_dim,
 * value_dim = n_v_heads*head_v_dim and conv_dim = 2*key_dim + value_dim are
 * derived. Layer L is full attention iff (L+1) % full_attn_interval == 0. */
typedef struct {
    uint32_t n_layers, n_heads, n_kv_heads, head_dim, hidden, ffn_hidden, vocab;
    float rope_theta, rms_eps;
    bool tied_embeddings;
    uint32_t rope_dim;
    uint32_t full_attn_interval;
    uint32_t n_k_heads, n_v_heads, head_k_dim, head_v_dim, conv_kernel;
    bool attn_output_gate;
} sg_cfg;

/* Per-layer weight pointers (surge.h:269-277). Exactly one of the two mixer
 * groups is non-NULL on a layer. GGUF dtypes: matmuls Q8_0 (or F32), every
 * small tensor F32. */
typedef struct {
    const void *q_proj, *k_proj, *v_proj, *o_proj, *q_norm, *k_norm,
               *gate_proj, *up_proj, *down_proj, *ln1, *ln2;
    const void *ssm_in_qkv, *ssm_in_z, *ssm_in_b, *ssm_in_a, *ssm_a,
               *ssm_dt_bias, *ssm_conv1d, *ssm_norm, *ssm_out;
} sg_layer_w;

/* What ssm_a stores (surge.h:281-284). GGUF stores -exp(A_log). */
typedef enum { SG_SSM_A_LOG = 0, SG_SSM_A_NEG_EXP = 1 } sg_ssm_a_form;

/* The model (surge.h:286-330). lm_head == tok_emb when tied. */
typedef struct {
    sg_cfg cfg;
    const void *tok_emb, *out_norm, *lm_head;
    sg_layer_w *layers;
    sg_tensor_type wtype;
    sg_ssm_a_form ssm_a_form;
    bool v_heads_tiled;
    sg_tensor_type ssm_a_type;
    sg_tensor_type ssm_norm_type;
    sg_tensor_type dense_type;
    bool norms_are_residual;
} sg_model;

/* Value-head -> key-head map (surge.h:337-343): GGUF tiles (h % n_k). */
static inline uint32_t sg_ssm_k_head(uint32_t v_head, uint32_t n_k_heads,
                                     uint32_t n_v_heads, bool tiled) {
    if (n_k_heads == 0 || n_v_heads < n_k_heads) return 0;
    return tiled ? (v_head % n_k_heads) : (v_head / (n_v_heads / n_k_heads));
}

/* Maps a qwen35/qwen3_5 GGUF onto an sg_model (surge.h:345). The model's
 * pointers alias the GGUF mapping, which must outlive it. */
sg_err sg_model_from_gguf(const sg_gguf *g, sg_model *m);
void sg_model_free(sg_model *m);                                     /* surge.h:347 */

/* ---------------------------------------------------------------------
 * GPU layer (surge.h:640-1408), implemented with HIP on gfx950
 * ---------------------------------------------------------------------
 *
 * Every sg_gpu_run_* entry point is synchronous: it launches on the
 * library's stream and waits. All buffers are f32 unless stated; a buffer
 * argument is a handle from sg_gpu_alloc / sg_gpu_wrap / sg_gpu_wrap_device.
 *
 * sg_gpu_run_op kernels and params (surge.h:666-707):
 *   kernel            a                     b                    out
 *   k_rmsnorm         x[n]                  w[n] (or NULL)       x'[n]
 *                     p: [0]=n [1]=eps bits [2]=1 if b holds w
 *   k_rmsnorm_heads   x[heads*stride]       w[n] or NULL         x'[heads*stride]
 *                     p: [0]=n [1]=heads [2]=eps bits [3]=stride (0 = n) [4]=1 if w
 *   k_rope            x[head_dim]           cos[half]|sin[half]  x'[head_dim]
 *                     p: [0]=head_dim [1]=rope_dim
 *   k_rope_heads      x[heads*stride]       cos|sin              x'
 *                     p: [0]=head_dim [1]=rope_dim [2]=heads [3]=stride
 *   k_matvec_q8       w Q8_0 rows*(cols/32) blocks   x[cols]     y[rows]
 *   k_matvec_f32      w[rows*cols]          x[cols]              y[rows]
 *                     p: [0]=rows [1]=cols (cols % 32 == 0 for q8)
 *   k_softmax         x[n]                  -                    p[n]
 *   k_swiglu          gate[n]               up[n]                silu(gate)*up
 *   k_silu            x[n]                  -                    silu(x)
 *   k_gate_sigmoid    x[n]                  gate[n]              x*sigmoid(gate)
 *   k_add             x[n]                  r[n]                 x+r
 *   k_scale           x[n]                  -                    x*scale  p: [1]=scale bits
 *   k_kv_store_f16    x[n] f32              -                    cache f16, p: [0]=n [1]=dst offset (elements)
 *   k_conv1d_step     x[channels]           w[channels*ksize]    y[channels] | state[(ksize-1)*channels]
 *                     p: [0]=channels [1]=ksize
 *   k_delta_step      S[dv*dk] in/out       q[dk]|k[dk]|v[dv]    y[dv]
 *                     p: [0]=dk [1]=dv [2]=beta bits [3]=decay bits
 *   k_rmsnorm_gated   y[heads*dv]           z[heads*dv] | w[dv]  silu(z)*rmsnorm(y,w)
 *                     p: [0]=dv [1]=heads [2]=eps bits
 *   k_matmul_q8       X[N*K] f32            W Q8_0 M*(K/32)      Y[N*M] f32
 *                     p: [0]=N [1]=M [2]=K
 *   k_argmax          v[n] f32              -                    u32 index (no reference
 *                     counterpart: the greedy loop's device argmax, = sg_argmax_f32)
 * Aliasing: out must not overlap a or b, except k_conv1d_step's state tail
 * and k_delta_step's in-place S (surge.h:709-712). */
typedef struct sg_gpu sg_gpu;

sg_err sg_gpu_init(sg_gpu **out);                                    /* surge.h:725 */
void sg_gpu_free(sg_gpu *g);                                         /* surge.h:726 */
sg_err sg_gpu_wrap(sg_gpu *g, const void *ptr, uint64_t nbytes, void **buf_out); /* surge.h:742 */
sg_err sg_gpu_alloc(sg_gpu *g, uint64_t nbytes, void **buf_out, void **host_out); /* surge.h:746 */
void sg_gpu_buf_free(void *buf);                                     /* surge.h:747 */
void *sg_gpu_buf_host(void *buf);                                    /* surge.h:749 */
uint64_t sg_gpu_current_alloc_bytes(const sg_gpu *g);                /* surge.h:756 */

/* Additions for discrete memory (no reference counterpart): wrap existing
 * device memory with no copy and no mirror; read a handle's device address;
 * explicit mirror synchronisation. */
sg_err sg_gpu_wrap_device(sg_gpu *g, void *dev_ptr, uint64_t nbytes, void **buf_out);
void *sg_gpu_buf_device(void *buf);
sg_err sg_gpu_buf_upload(void *buf);
sg_err sg_gpu_buf_download(void *buf);

sg_err sg_gpu_run_op(sg_gpu *g, const char *kernel, void *a, void *b, void *out,
                     const uint32_t params[8]);                      /* surge.h:761 */

/* fp16-KV single-pass decode attention (surge.h:774). q f32 [n_heads,
 * q_stride]; k, v f16 [seq, n_kv, hd]; out f32 [n_heads, hd].
 * p: [0]=n_heads [1]=n_kv [2]=hd [3]=seq [4]=q_stride [5]=scale bits. */
sg_err sg_gpu_run_attn_decode_f16(sg_gpu *g, void *q, void *k, void *v, void *out,
                                  const uint32_t params[8]);
/* No reference counterpart: sg_gpu_run_attn_decode_f16 with no device
 * allocation, for callers that cannot allocate (serving loops, harnesses
 * that forbid hipMalloc). Its partials live in a static 4 MiB device
 * workspace per GPU, so n_heads * n_splits * (head_dim + 2) * 4 bytes must
 * fit (n_splits = sg_gpu_splitk_gqa_n_splits(seq)); larger calls are refused.
 * Like every sg_gpu_run_* call it is synchronous (it uploads and downloads
 * the buffers' host mirrors and waits for the library's stream), so it
 * cannot be recorded into a HIP graph capture of that stream. Calls that
 * overlap on one GPU share the workspace and race. */
sg_err sg_gpu_run_attn_decode_f16_noalloc(sg_gpu *g, void *q, void *k, void *v, void *out,
                                          const uint32_t params[8]);

/* Split-K decode attention (surge.h:890-980). Split i covers
 * [i*seq/n, (i+1)*seq/n); m, s f32 [n_heads, n_splits]; acc f32
 * [n_heads, n_splits, hd]. p: [0]=n_heads [1]=n_kv [2]=hd [3]=seq
 * [4]=q_stride [5]=scale bits [6]=n_splits. The per-head and GQA partials
 * produce the same bytes here (one kernel serves both). */
sg_err sg_gpu_run_attn_splitk_partial(sg_gpu *g, void *q, void *k, void *v,
                                      void *m, void *s, void *acc,
                                      const uint32_t params[8]);
sg_err sg_gpu_run_attn_splitk_partial_gqa(sg_gpu *g, void *q, void *k, void *v,
                                          void *m, void *s, void *acc,
                                          const uint32_t params[8]);
sg_err sg_gpu_run_attn_splitk_combine(sg_gpu *g, void *m, void *s, void *acc,
                                      void *out, const uint32_t params[8]);

/* The online-softmax partial (surge.h:974-980): the partial kernel here is
 * the online form already, so this one-shot is the GQA one and gives its
 * bytes (the reference's online kernel differs from its four-pass one in the
 * last bits). */
sg_err sg_gpu_run_attn_splitk_partial_gqa_online(sg_gpu *g, void *q, void *k, void *v,
                                                 void *m, void *s, void *acc,
                                                 const uint32_t params[8]);

/* Causal chunk attention (surge.h:787-788): q f32 [n, n_heads, q_stride];
 * k, v f16 [base+n, n_kv, hd] already holding base+n positions; out f32
 * [n, n_heads, hd]; token t (position base+t) attends over 0..base+t.
 * p: [0]=n_heads [1]=n_kv [2]=hd [3]=base [4]=n [5]=q_stride [6]=scale bits. */
sg_err sg_gpu_run_attn_prefill(sg_gpu *g, void *q, void *k, void *v, void *out,
                               const uint32_t params[8]);

/* Decode attention selection (surge.h:1011-1106, 1179-1254). Read at
 * sg_gpu_state_new:
 *   SURGE_KV_DTYPE           f16 (default); f32 is refused (no f32 cache is
 *                            built); anything else warns and keeps f16;
 *   SURGE_ATTN_SPLITK        1 (default) split-K; 0 one split per head (the
 *                            single-pass form, counted in neither counter);
 *   SURGE_ATTN_SPLITK_GQA    1 (default) the partial shared by a GQA group
 *                            (group in [2, 8]); 0 the per-head partial (same
 *                            bytes); unrecognised values warn, keep 1;
 *   SURGE_ATTN_SPLITK_ONLINE exactly 0 (default) or 1, else refused; 1 counts
 *                            the dispatches as the online arm (same kernel:
 *                            the partial is the online form) and the GQA
 *                            predicate then answers false;
 *   SURGE_SPLITK_GQA_CAP     the split cap, plain digits in [4, 1024]
 *                            (unset: one partial workgroup per CU,
 *                            CUs / n_kv_heads within [4, 128]).
 * The arm is fixed per state: the MI355X policy has no occupancy floor, so
 * `seq` does not change the answers. The counters count what sg_gpu_forward
 * and sg_gpu_decode_greedy encoded since the last sg_gpu_state_new, one per
 * attention layer per step; one-shots are not counted. */
uint32_t sg_gpu_splitk_n_splits(uint32_t seq);                     /* surge.h:1106 */
uint32_t sg_gpu_splitk_gqa_n_splits(uint32_t seq);                 /* surge.h:1081 */
uint32_t sg_gpu_splitk_gqa_n_splits_at(const sg_gpu *g, uint32_t seq); /* surge.h:1104 */
uint32_t sg_gpu_splitk_gqa_cap(const sg_gpu *g);                   /* surge.h:1105 */
bool sg_gpu_splitk_gqa_selected(const sg_gpu *g, uint32_t n_heads,
                                uint32_t n_kv_heads, uint32_t seq); /* surge.h:1020 */
void sg_gpu_splitk_dispatch_counts(const sg_gpu *g, uint64_t *per_head, uint64_t *gqa); /* surge.h:1022 */
bool sg_gpu_splitk_online_selected(const sg_gpu *g, uint32_t n_heads,
                                   uint32_t n_kv_heads, uint32_t head_dim,
                                   uint32_t seq);                   /* surge.h:1047 */
uint64_t sg_gpu_splitk_online_dispatches(const sg_gpu *g);          /* surge.h:1050 */

/* DeltaNet one-shots (surge.h:1133-1142). k_delta_multi: S [n_v, dv, dk]
 * in/out, qkv [conv_dim] (post conv+silu, pre norm), out [value_dim], gates
 * [2*n_v] = beta[n_v] | decay[n_v]. p: [0]=dk [1]=dv [2]=n_v [3]=n_k
 * [4]=key_dim [5]=tiled. q/k arrive already normalised and scaled, as in the
 * reference's k_delta_multi (kernels.metal:764-805). */
sg_err sg_gpu_run_delta_multi(sg_gpu *g, void *S, void *qkv, void *out, void *gates,
                              const uint32_t params[8]);
/* The decode path's fused DeltaNet layer step on caller buffers (no
 * reference counterpart: the reference's decode kernels k_conv1d_step,
 * k_delta_gates, k_delta_multi and k_rmsnorm_gated are one kernel here).
 *   in    [conv_dim + value_dim + 2 n_v]   qkv (before the conv) | z | b | a
 *   w     [conv_dim ksize + 2 n_v + dv]    conv_w | ssm_a | dt_bias | ssm_norm
 *   state [(ksize-1) conv_dim + n_v dv dk] conv tail (oldest first) | S, in/out
 *   out   [value_dim]                      silu(z) * rmsnorm(y, ssm_norm)
 * p: [0]=dk [1]=dv [2]=n_v [3]=n_k [4]=ksize [5]=tiled [6]=ssm_a is -exp(A_log)
 * [7]=eps bits; conv_dim = 2 n_k dk + n_v dv; dv <= 128. */
sg_err sg_gpu_run_gdn_step(sg_gpu *g, void *in, void *w, void *state, void *out,
                           const uint32_t params[8]);
/* The prefill path's DeltaNet layer core over a chunk of n tokens (the chunk
 * conv with its q/k norm, the conv ring, the gates, the delta-rule scan in
 * the build's default form, the RMSNormGated rows), with no reference
 * counterpart (the reference's prefill loops its per-token kernels,
 * kernels.metal:1111-1278). Buffers as sg_gpu_run_gdn_step with n rows: in
 * [n][conv_dim + value_dim + 2 n_v], out [n][value_dim]; w and state the
 * same. p: [0]=dk [1]=dv [2]=n_v [3]=n_k [4]=ksize [5]=flags (bit 0 tiled,
 * bit 1 ssm_a is -exp(A_log), bits 2-3 the first position mod 4) [6]=n
 * [7]=eps bits. */
sg_err sg_gpu_run_gdn_chunk(sg_gpu *g, void *in, void *w, void *state, void *out,
                            const uint32_t params[8]);
/* The prefill path's attention layer core over a chunk of n tokens at
 * positions base .. base+n-1 (q_norm / k_norm, partial RoPE, f16 K/V store,
 * the flash pass with its key split and combine, sigmoid output gate), with
 * no reference counterpart (the reference's prefill runs its attention
 * kernels per token, kernels.metal:1021-1081). in [n][n_heads 2 hd + 2 n_kv
 * hd] (per query head q | gate, then k, then v), w [2 hd] q_norm | k_norm,
 * kv [2][base + n][n_kv][hd] f16 (K then V; positions below base given, the
 * chunk's written), out [n][n_heads hd]. p: [0]=n_heads [1]=n_kv [2]=hd (64,
 * 128 or 256) [3]=rope_dim [4]=base [5]=n [6]=rope_theta bits [7]=eps bits.
 * The attention scale is fixed at 1/sqrt(hd), as the model's decode and
 * prefill use it (ref.c:1238); params has no slot left for another. */
sg_err sg_gpu_run_attn_chunk(sg_gpu *g, void *in, void *w, void *kv, void *out,
                             const uint32_t params[8]);
/* Prefill chunk hooks (surge.h:1111-1142), reference layouts:
 *   conv1d_chunk: x [n_tok, ch], w [ch, ksize], out [n_tok, ch], state
 *     [ksize-1, ch] oldest-first in/out; no activation. p: [0]=ch [1]=ksize [2]=n_tok
 *   delta_gates_chunk: a, b [n_tok, n], gates [n_tok, 2n] (beta | decay),
 *     adt [ssm_a(n) | dt_bias(n)]. p: [0]=n [1]=neg_exp [2]=n_tok
 *   delta_chunk: S [n_v, dv, dk] in/out, qkv [n_tok, conv_dim] (normalised
 *     q, k), out [n_tok, value_dim], gates [n_tok, 2*n_v].
 *     p: [0]=dk [1]=dv [2]=n_v [3]=n_k [4]=key_dim [5]=tiled [6]=n_tok [7]=conv_dim
 *   rmsnorm_gated_chunk: y, z, out [n_tok, heads*dv], w [dv].
 *     p: [0]=dv [1]=heads [2]=eps bits [3]=n_tok */
sg_err sg_gpu_run_conv1d_chunk(sg_gpu *g, void *x, void *w, void *out, void *state,
                               const uint32_t params[8]);
sg_err sg_gpu_run_delta_gates_chunk(sg_gpu *g, void *a, void *b, void *gates, void *adt,
                                    const uint32_t params[8]);
sg_err sg_gpu_run_delta_chunk(sg_gpu *g, void *S, void *qkv, void *out, void *gates,
                              const uint32_t params[8]);
sg_err sg_gpu_run_rmsnorm_gated_chunk(sg_gpu *g, void *y, void *z, void *out, void *w,
                                      const uint32_t params[8]);

/* Decode (surge.h:1260-1274). */
sg_err sg_gpu_load_model(sg_gpu *g, const sg_model *m);
sg_err sg_gpu_state_new(sg_gpu *g, const sg_model *m, uint32_t max_ctx);
void sg_gpu_state_reset(sg_gpu *g);
sg_err sg_gpu_forward(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos,
                      const float **logits);
uint32_t sg_gpu_used(const sg_gpu *g);

/* Chunked prefill (surge.h:1306-1309). */
#define SG_PREFILL_CHUNK_DEFAULT 1024u
sg_err sg_gpu_prefill(sg_gpu *g, const sg_model *m, const int32_t *tokens,
                      uint32_t n_tokens, uint32_t chunk_size,
                      const float **out_last_logits);
/* Apple compositor mitigations (surge.h:1372-1408): kept for API
 * compatibility; no-ops on MI355X (nothing to yield to). */
void sg_gpu_set_prefill_rest(sg_gpu *g, uint32_t work_budget_ms, uint32_t rest_ms);
uint64_t sg_gpu_prefill_rest_ms(const sg_gpu *g);
void sg_gpu_set_prefill_max_burst(sg_gpu *g, uint32_t max_burst_ms);
uint64_t sg_gpu_prefill_segments(const sg_gpu *g);

/* Device-resident greedy argmax over the last forward's logits (no
 * reference counterpart; the reference reads host logits). Lowest index wins
 * an exact tie, as sg_argmax_f32. */
sg_err sg_gpu_argmax(sg_gpu *g, uint32_t *token_out);
/* Forward without the logits download (no reference counterpart): for
 * callers that only need sg_gpu_argmax or time the step. */
sg_err sg_gpu_forward_nosync(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos);
sg_err sg_gpu_sync(sg_gpu *g);
/* Device-resident greedy decode (no reference counterpart): feeds `token` at
 * `pos`, then keeps choosing the next token by argmax on the device for
 * n_steps steps with no host round trip; out_tokens[i] is the argmax after
 * step i. Same tokens as calling sg_gpu_forward + sg_argmax_f32 in a loop. */
sg_err sg_gpu_decode_greedy(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos,
                            uint32_t n_steps, int32_t *out_tokens);
/* The same with per-token timestamps (no reference counterpart): t_cum[i] is
 * the seconds from just before the first step to the end of step i, from HIP
 * events between the steps, the series sg_bench_slope fits. */
sg_err sg_gpu_decode_greedy_timed(sg_gpu *g, const sg_model *m, int32_t token, uint32_t pos,
                                  uint32_t n_steps, int32_t *out_tokens, double *t_cum);
/* Decode at depth without a prefill (no reference counterpart; for
 * benchmarks of the KV read path at long context): fills every attention
 * layer's K/V cache rows [0, n_tokens) with seeded f16 values in [-2, 2], the
 * DeltaNet states and conv rings with seeded values in [-0.05, 0.05], and
 * sets the state's position to n_tokens (< max_ctx). The next call is then
 * sg_gpu_forward / sg_gpu_decode_greedy at pos = n_tokens. Same seed, same
 * state. */
sg_err sg_gpu_state_fill_synthetic(sg_gpu *g, uint32_t n_tokens, uint32_t seed);

/* Measurement hooks (no reference counterpart): the library's HIP stream
 * (a hipStream_t) for event timing, and one decode-step GEMV enqueued alone
 * against the live state (which: 0 input projection, 1 output projection,
 * 2 gate/up, 3 down, 4 lm_head). */
void *sg_gpu_stream(const sg_gpu *g);
sg_err sg_gpu_enqueue_gemv(sg_gpu *g, uint32_t layer, uint32_t which);
/* The same with the GEMV's measurement overrides: tune_r rows per wave of
 * the row-group kernel (1, 2 or 4) and tune_blocks its workgroup count (0:
 * the launch policy). */
sg_err sg_gpu_enqueue_gemv_tuned(sg_gpu *g, uint32_t layer, uint32_t which, uint32_t tune_r, uint32_t tune_blocks);

/* Timing hooks for the per-kernel micro configs (no reference counterpart).
 * Each runs one product kernel `reps` times back to back and reports the
 * average microseconds per launch from HIP events around the launches;
 * launch i reads input copy i mod n of n copies spanning at least
 * rotate_bytes (0: one copy, cache resident), so timed launches do not find
 * their inputs in the 256 MB MALL.
 *   sg_gpu_time_matvec_q8: the decode GEMV on a Q8_0 [rows][cols/32] matrix;
 *   sg_gpu_time_attn: the split-K partial (q as given) then the LSE combine,
 *     p as sg_gpu_run_attn_splitk_partial_gqa (p[6] = 0: the decode policy's
 *     split count); us[0] partial, us[1] combine;
 *   sg_gpu_time_gdn_step: the fused DeltaNet step, in/w/p as
 *     sg_gpu_run_gdn_step, the state S and conv ring rotated. */
sg_err sg_gpu_time_matvec_q8(sg_gpu *g, void *w, void *x, void *y, uint32_t rows, uint32_t cols,
                             uint64_t rotate_bytes, uint32_t reps, double *us);
sg_err sg_gpu_time_attn(sg_gpu *g, void *q, void *k, void *v, void *out, const uint32_t params[8],
                        uint64_t rotate_bytes, uint32_t reps, double *us);
sg_err sg_gpu_time_gdn_step(sg_gpu *g, void *in, void *w, void *out, const uint32_t params[8],
                            uint64_t rotate_bytes, uint32_t reps, double *us);
/* The floors under every decode kernel (no reference counterpart): a plain
 * streaming read of `bytes` (multiple of 16) by 1024 workgroups, with the
 * same input rotation as above; and `reps` empty kernels launched one by one
 * (graph = 0) or replayed from one captured HIP graph (graph != 0). Average
 * microseconds per launch. */
sg_err sg_gpu_time_read(sg_gpu *g, uint64_t bytes, uint64_t rotate_bytes, uint32_t reps, double *us);
sg_err sg_gpu_time_empty(sg_gpu *g, uint32_t reps, int graph, double *us);
/* The sequential-launch floor of one greedy decode token (no reference
 * counterpart): the loaded model's decode launch sequence at `ctx` keys, in
 * its order (embedding; per layer the input projection, attention partial and
 * combine or DeltaNet step, output projection, gate/up, down; lm_head, two
 * argmax passes, step advance), captured in one HIP graph with every kernel
 * replaced by a plain streaming read of that kernel's algorithmic bytes
 * (mode 1, each read from its own region of a buffer of the token's total, so
 * nothing is served from the MALL) or by an empty kernel (mode 0), and
 * replayed `reps` times; mode 2 launches the same reads one by one without a
 * graph (for kernel traces). Average microseconds per token; n_kernels and bytes
 * (either may be NULL) get the launch count and the token's summed bytes.
 * Needs a Q8_0 model and a state; mode 1 allocates the token's bytes. */
sg_err sg_gpu_time_floor(sg_gpu *g, uint32_t ctx, uint32_t mode, uint32_t reps, double *us, uint32_t *n_kernels,
                         uint64_t *bytes);
/* The prefill GEMM (no reference counterpart) on one of the loaded model's
 * weights (which: 0 input projection with its RMSNorm, 1 output projection
 * += into the residual rows, 2 gate/up with RMSNorm and SwiGLU, 3 down +=)
 * for a chunk of n tokens of synthetic activations, as the chunked prefill
 * launches it (split, MFMA tiles, split-K reduce): `reps` back-to-back
 * products, average microseconds per product. Needs a live state; it
 * overwrites the state's prefill scratch. */
sg_err sg_gpu_time_gemm(sg_gpu *g, uint32_t layer, uint32_t which, uint32_t n, uint32_t reps, double *us);

/* ---------------------------------------------------------------------
 * KV cache + DeltaNet state sizing and f16 (surge.h:1410-1501)
 * --------------------------------------------------------------------- */
#define SG_KV_CAP_DEFAULT 131072u
#define SG_KV_CAP_MAX     262144u
uint64_t sg_kv_bytes(const sg_cfg *c, uint32_t cap, sg_tensor_type dtype); /* surge.h:1456 */
uint64_t sg_kv_state_bytes(const sg_cfg *c);                               /* surge.h:1457 */
uint16_t sg_f32_to_f16(float f);                                           /* surge.h:1463 */
float    sg_f16_to_f32(uint16_t h);                                        /* surge.h:1464 */

/* The KV / DeltaNet-state allocation module (surge.h:1466-1501). Buffers come
 * from an injected backend; sg_gpu_init registers sg_gpu_alloc,
 * sg_gpu_buf_free and sg_gpu_buf_host (reference metal.m:627-633). The alloc
 * must zero-fill. A full-attention layer has separate K and V of
 * [cap, n_kv_heads, head_dim] in kv_dtype (f16 or f32); a DeltaNet layer a
 * conv tail [conv_kernel-1, conv_dim] and S [n_v_heads, head_v_dim,
 * head_k_dim] in f32. cap 0 means SG_KV_CAP_DEFAULT; above SG_KV_CAP_MAX is
 * refused. sg_kv_reset zeroes the conv tails and S through their host views
 * and leaves K/V; sg_kv_advance refuses to pass cap. The getters return NULL
 * for the other kind of layer or a layer out of range. */
typedef struct sg_kv sg_kv;
typedef sg_err (*sg_kv_alloc_fn)(sg_gpu *g, uint64_t nbytes, void **buf, void **host);
typedef void   (*sg_kv_free_fn)(void *buf);
typedef void  *(*sg_kv_host_fn)(void *buf);
void sg_kv_set_backend(sg_kv_alloc_fn alloc, sg_kv_free_fn free_, sg_kv_host_fn host); /* surge.h:1474 */
sg_err sg_kv_new(sg_gpu *g, const sg_cfg *c, uint32_t cap,
                 sg_tensor_type kv_dtype, sg_kv **out);            /* surge.h:1481 */
void sg_kv_free(sg_kv *kv);                                        /* surge.h:1483 */
void sg_kv_reset(sg_kv *kv);                                       /* surge.h:1487 */
sg_err sg_kv_advance(sg_kv *kv, uint32_t n);                       /* surge.h:1491 */
uint32_t sg_kv_used(const sg_kv *kv);                              /* surge.h:1492 */
uint32_t sg_kv_cap(const sg_kv *kv);                               /* surge.h:1493 */
void *sg_kv_k(const sg_kv *kv, uint32_t layer);                    /* surge.h:1498 */
void *sg_kv_v(const sg_kv *kv, uint32_t layer);                    /* surge.h:1499 */
void *sg_kv_conv(const sg_kv *kv, uint32_t layer);                 /* surge.h:1500 */
void *sg_kv_s(const sg_kv *kv, uint32_t layer);                    /* surge.h:1501 */

/* ---------------------------------------------------------------------
 * Greedy argmax (surge.h:1503-1512): lowest index wins an exact tie.
 * --------------------------------------------------------------------- */
uint32_t sg_argmax_f32(const float *v, uint32_t n);

/* ---------------------------------------------------------------------
 * Bench math (surge.h:1784-1824)
 * --------------------------------------------------------------------- */
double sg_bench_slope(const double *t_wall_cum, uint32_t n, uint32_t warmup);
double sg_bench_avg_tps(const double *t_wall_cum, uint32_t n, uint32_t warmup);
uint32_t sg_bench_default_warmup(uint32_t n_gen);

/* One surge-bench leaderboard row (surge.h:1845-1914), field for field: the
 * reference's CLI and recipes fill it and hand it to the formatters below.
 * Every char array is NUL-terminated by whoever fills it. */
typedef struct {
    char model[64];
    char engine[64];
    double prefill_tps;          /* < 0: not measured ("-" in the md row) */
    double decode_tps_slope;     /* sg_bench_slope */
    double decode_tps_avg;       /* sg_bench_avg_tps */
    double prefill_wall_s;
    double decode_wall_s;
    unsigned long long prefill_segments;
    double prefill_rest_s;
    double prefill_compute_tps;
    double decode_rest_s;
    double decode_compute_tps;
    uint32_t decode_rests;
    uint32_t decode_clamp_events;
    double decode_baseline_ms;
    double peak_ram_gib;
    double gpu_alloc_gib;
    uint32_t recall_hits;
    uint32_t recall_total;
    uint32_t assoc_hits;
    uint64_t n_prompt_tok;
    uint32_t n_gen;
    double wall_s;
    double gemm_tflops;
    bool ingestion_ok;
    char status[16];             /* "DONE" or "VOID", set by sg_bench_finalize_status */
    char log_id[96];
} sg_bench_row;

/* | model | engine | prefill t/s | decode t/s | peak RAM | recall | wall | status |
 * with prefill "%.0f" (or "-" below 0), decode slope "%.2f", "%.1f GiB",
 * "hits/total", wall in whole minutes, status (surge.h:1916-1924). */
void sg_bench_format_md_row(const sg_bench_row *row, char *buf, size_t cap); /* surge.h:1924 */
/* A flat JSON object of every field under its field name: numbers "%.6g",
 * ingestion_ok a JSON bool, strings JSON-escaped (quote, backslash, control
 * bytes as \u00XX); truncated to cap like the md row (surge.h:1926-1937). */
void sg_bench_format_json(const sg_bench_row *row, char *buf, size_t cap);   /* surge.h:1937 */
#define SG_BENCH_GEMM_MIN_TFLOPS 20.5
/* Admitted iff gemm_tflops > SG_BENCH_GEMM_MIN_TFLOPS and ingestion_ok;
 * finalize sets status to "DONE" or "VOID" accordingly (surge.h:1939-1955). */
bool sg_bench_admitted(const sg_bench_row *row);                           /* surge.h:1950 */
void sg_bench_finalize_status(sg_bench_row *row);                          /* surge.h:1955 */
/* The ingestion guard (surge.h:1980-1993): *ok = n_ids <= max_ctx (nothing
 * truncated) and expect_min <= n_ids <= expect_max (the prompt's id count is
 * the one expected); logged to stderr; a NULL ok is a no-op. */
void sg_bench_check_ingestion(uint64_t n_ids, uint32_t max_ctx, uint64_t expect_min,
                              uint64_t expect_max, bool *ok);                /* surge.h:1992 */

/* The peak-memory probe (surge.h:2104-2142). sg_proc_phys_footprint: the
 * process's resident host memory in bytes, here from Linux's
 * /proc/self/statm (resident pages x page size; the reference reads
 * Mach's phys_footprint); 0, with a message on stderr, when it cannot be
 * read. sg_mem_tracker: a running maximum of two signals sampled together,
 * peak = max(peak, current_alloc, phys_footprint); reset zeroes it, a NULL
 * tracker is a no-op and reads back 0. */
uint64_t sg_proc_phys_footprint(void);                                     /* surge.h:2128 */
typedef struct { uint64_t peak; } sg_mem_tracker;                          /* surge.h:2138 */
void sg_mem_tracker_reset(sg_mem_tracker *t);                              /* surge.h:2139 */
void sg_mem_tracker_sample(sg_mem_tracker *t, uint64_t current_alloc,      /* surge.h:2140 */
                           uint64_t phys_footprint);
uint64_t sg_mem_tracker_peak(const sg_mem_tracker *t);                     /* surge.h:2141 */

/* ---------------------------------------------------------------------
 * Synthetic random-init models (no reference counterpart: the reference
 * writes its fixtures from Python, tools/make_fixtures.py:1242-1416).
 * ---------------------------------------------------------------------
 * Builds a qwen35-shaped model of the given config with seeded random
 * weights, laid out in one host allocation exactly as a GGUF file would hold
 * them (Q8_0 matmuls with 34-byte blocks, F32 small tensors, -exp(A_log)
 * ssm_a, absolute norms near 1, tiled value heads). Deterministic for a
 * seed regardless of thread count. sg_synth_write_gguf writes the same
 * model as a GGUF v3 file that sg_gguf_open + sg_model_from_gguf read back.
 * wtype is SG_T_Q8_0 or SG_T_F32. */
typedef struct sg_synth sg_synth;
sg_err sg_synth_new(const sg_cfg *c, sg_tensor_type wtype, uint64_t seed,
                    sg_synth **out);
const sg_model *sg_synth_model(const sg_synth *s);
uint64_t sg_synth_bytes(const sg_synth *s);
sg_err sg_synth_write_gguf(const sg_synth *s, const char *path);
void sg_synth_free(sg_synth *s);

#ifdef __cplusplus
}
#endif
#endif /* SURGE_H */
