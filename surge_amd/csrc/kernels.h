/* kernels.h - launchers exported by kernels.hip to the C host layer (hip.c).
 *
 * Every launcher is asynchronous on the given stream and takes device
 * pointers only. Shapes are validated by the caller (hip.c) before any launch:
 * the kernels trust them. Q8_0 matrices live on the device in a split layout
 * built at load time by sgk_repack_q8: an int8 plane qs[rows][cols] (each row
 * 32-byte aligned, so a lane can stream 16 bytes per load) and an f16 scale
 * plane d[rows][cols/32]. The bytes per weight are the same as the file's
 * 34-byte blocks.
 */
#ifndef SURGE_KERNELS_H
#define SURGE_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The DeltaNet descriptor's pointers are typed as global-memory pointers in
 * the device compile pass, so their loads and stores are global ones rather
 * than flat ones (a flat access also counts against the LDS wait counter,
 * which would make LDS reads wait for memory). Same bits and layout as the
 * host's plain pointers. */
#if defined(__HIP_DEVICE_COMPILE__)
#define SGK_G __attribute__((address_space(1)))
#else
#define SGK_G
#endif

/* Per-token step descriptor, read by every position-dependent kernel so one
 * captured HIP graph serves every decode step. */
typedef struct {
    int32_t token;
    uint32_t pos;       /* position being written; attention sees pos+1 keys */
    uint32_t pad[2];
} sgk_step;

/* The split-K decode-attention split count (also evaluated on the device).
 * MI355X policy: about 64 keys per split (one key tile of the partial kernel
 * at head_dim 256), capped; never more splits than keys. A decode state's
 * cap defaults to one partial workgroup per CU (n_splits * n_kv_heads <=
 * CUs, at most SGK_MAX_SPLITS): on the 27B shape (4 kv heads) 64 splits
 * beat 128 (two workgroups per CU) at every depth measured from 8k to 262k
 * keys, and a count just past one per CU (65 at 4097 keys) cost a second
 * pass. The state-free count (sgk_n_splits) keeps the SGK_MAX_SPLITS cap. */
#define SGK_MAX_SPLITS 128u
#define SGK_KEYS_PER_SPLIT 64u
/* A state may lower or raise the cap (SURGE_SPLITK_GQA_CAP) within [4, 1024]. */
#define SGK_SPLIT_CAP_MIN 4u
#define SGK_SPLIT_CAP_MAX 1024u
static inline uint32_t sgk_n_splits_cap(uint32_t seq, uint32_t cap) {
    uint32_t n = (seq + SGK_KEYS_PER_SPLIT - 1) / SGK_KEYS_PER_SPLIT;
    if (n < 1) n = 1;
    if (n > cap) n = cap;
    return n;
}
static inline uint32_t sgk_n_splits(uint32_t seq) { return sgk_n_splits_cap(seq, SGK_MAX_SPLITS); }

/* GEMV prologues (what is staged into LDS as the input vector: x, or x*w with
 * the RMS factor applied to each row sum) and epilogues (what is done with
 * each output row). */
enum { SGK_PRO_NONE = 0, SGK_PRO_RMS = 1, SGK_PRO_GATED = 2 };
#define SGK_GATED_MAX_HEADS 256u    /* value heads the gated prologue takes */
enum { SGK_EPI_STORE = 0, SGK_EPI_ADD = 1, SGK_EPI_SWIGLU = 2,
       SGK_EPI_TILE = 3, SGK_EPI_SWIGLU_XS = 4 /* prefill GEMM internal */ };

typedef struct {
    const int8_t *qs;       /* Q8: int8 plane [rows][cols] */
    const uint16_t *d;      /* Q8: f16 scales [rows][cols/32] */
    const float *wf;        /* F32 weights [rows][cols] (when qs == NULL) */
    uint32_t rows, cols;
    const float *x;         /* input vector [cols], 16-byte aligned */
    const float *nw;        /* PRO_RMS norm weight [cols], 16-byte aligned */
    float eps;
    float *y;               /* output [rows] (or [rows/2] for SWIGLU) */
    int pro, epi;
    uint32_t tune_r, tune_blocks;   /* 0 = default; rows per wave (1/2/4), workgroups */
    /* PRO_GATED (the DeltaNet out projection after a step of SGK_GDN_BLOCKS
     * workgroups per head): x = silu(z) * (y * ssm_norm), gss = each head's
     * row-block sums of y^2 [heads][SGK_GDN_BLOCKS], gdv = head_v_dim; the
     * prologue stages x * rsqrt(mean y^2 + eps) per head */
    const float *gss;
    uint32_t gdv;
} sgk_gemv;

hipError_t sgk_gemv_launch(const sgk_gemv *a, hipStream_t s);

/* Split Q8_0 blocks (34-byte) of a [rows, cols] matrix into the device layout
 * (qs [ld][cols] int8, d [ld][cols/32] f16 scales) and, when dt is not NULL,
 * a block-major copy of the scales, dt [cols/32][ld], for the prefill GEMM.
 * Destination row of source row r is row0 + r * row_step; ld is the
 * destination matrix's row count. */
hipError_t sgk_repack_q8(const uint8_t *src, uint32_t rows, uint32_t cols,
                         int8_t *qs, uint16_t *d, uint16_t *dt, uint32_t ld, uint32_t row0,
                         uint32_t row_step, hipStream_t s);

/* Embedding row gather: x[hidden] = row `token` of the table (token from the
 * step descriptor when `step` is non-NULL, else `token`). */
hipError_t sgk_embed(const int8_t *qs, const uint16_t *d, const float *wf, uint32_t hidden,
                     const sgk_step *step, int32_t token, float *x, hipStream_t s);

/* Elementwise ops: out[i] = op(a[i], b[i]). */
enum { SGK_EW_SWIGLU = 0, SGK_EW_SILU, SGK_EW_GATE_SIGMOID, SGK_EW_ADD, SGK_EW_SCALE,
       SGK_EW_TO_F16 };
hipError_t sgk_elementwise(int op, const float *a, const float *b, void *out, uint32_t n,
                           float scale, hipStream_t s);

/* RMSNorm over `heads` slices of n elements at stride `stride` (out may
 * equal x). w may be NULL. */
hipError_t sgk_rmsnorm_heads(const float *x, const float *w, float *out, uint32_t n,
                             uint32_t heads, uint32_t stride, float eps, hipStream_t s);
/* Half-split partial RoPE over `heads` slices, cos|sin table cs[rope_dim]. */
hipError_t sgk_rope_heads(const float *x, const float *cs, float *out, uint32_t head_dim,
                          uint32_t rope_dim, uint32_t heads, uint32_t stride, hipStream_t s);
hipError_t sgk_softmax(const float *x, float *out, uint32_t n, hipStream_t s);

/* Decode attention over one token (a decode step) or many (a prefill chunk:
 * gridDim.z = ntok). Token z uses steps[z] (it writes K/V at steps[z].pos and
 * attends over pos+1 keys); q/gate of token z start at q + z*q_tok (head h at
 * + h*q_stride, its gate half at + hd); its m/s/acc slice starts at
 * z*n_heads*max_splits (x hd for acc); its output at out + z*out_tok.
 * Without steps (one-shot per-op calls) seq/n_splits are taken from here. */
#define SGK_PREFILL_SPLITS 8u
typedef struct {
    float *q;                   /* prep: the fused q|k|v GEMM rows (q normed+roped in place) */
    uint16_t *kc, *vc;          /* f16 caches (layout: kv_ps, kv_hs below) */
    float *m, *s, *acc;         /* partials */
    float *out;                 /* combine output [ntok][n_heads*hd] */
    const float *gate;          /* combine: q rows again (gate half), or NULL */
    const sgk_step *steps;
    uint32_t n_heads, n_kv, hd, rope_dim, q_stride, q_tok, out_tok;
    uint32_t seq, n_splits, max_splits, ntok;
    uint32_t split_cap;         /* decode split cap (0 = SGK_MAX_SPLITS) */
    float scale;
    int prefill;                /* split policy: 0 decode (kernels.h), 1 prefill */
    /* fused prep (decode, ntok == 1): q_norm/k_norm weights, the cos|sin
     * table [max_ctx][rope_dim], the norm eps */
    int fuse_prep;
    const float *qn, *kn, *cs;
    float eps;
    /* K/V cache strides in elements: position p of kv head h starts at
     * p*kv_ps + h*kv_hs. 0 = the reference layout [pos][n_kv][hd]
     * (kv_ps = n_kv*hd, kv_hs = hd); the decode state is head-major
     * [n_kv][cap][hd] (kv_ps = hd, kv_hs = cap*hd), so a split's keys are
     * one contiguous run. */
    uint32_t kv_ps;
    uint64_t kv_hs;
    /* Per-head partial (the reference's k_attn_decode_splitk_partial): one
     * workgroup per (split, query head) instead of per (split, kv head); the
     * grid's y is n_heads. Each head's arithmetic is the same as in the
     * group-shared form, so both give the same bytes. */
    int per_head;
} sgk_attn;

/* q_norm/k_norm + RoPE on each head, K and V stored f16 at each token's
 * position. cs_table is [max_ctx][rope_dim] (cos | sin per position). */
hipError_t sgk_attn_prep(const sgk_attn *a, const float *qn, const float *kn,
                         const float *cs_table, float eps, hipStream_t s);
/* Split-K GQA partials: workgroup (split, kv head, token) serves all
 * n_heads/n_kv query heads of the group (grid x = max_splits with steps).
 * With fuse_prep the prep above is done inside (q in LDS; the split holding
 * the position stores the new K/V), so a decode step needs no prep launch.
 * Without it q is used as given (already normed and roped) and nothing is
 * stored: the per-op one-shots run the decode kernel this way. */
hipError_t sgk_attn_partial(const sgk_attn *a, hipStream_t s);
/* LSE combine with the optional fused sigmoid output gate. */
hipError_t sgk_attn_combine(const sgk_attn *a, hipStream_t s);
/* Prefill: causal attention of a chunk (ntok tokens at consecutive positions
 * from steps[0].pos, prepped by sgk_attn_prep) in one MFMA pass per (64-token
 * block, head), gate applied, written to out. head_dim 64, 128 or 256. */
hipError_t sgk_attn_flash(const sgk_attn *a, hipStream_t s);

/* Gated DeltaNet decode step for one layer, fused: causal conv (ring state
 * of 4 slots indexed by position) + SiLU, q/k RMS (eps 1e-6) and scaling,
 * the beta/decay gates and the rank-1 state update with readout. Writes the
 * pre-norm readout y[value_dim]. The out-projection's gated-RMS prologue
 * finishes the layer. */
typedef struct {
    const float SGK_G *in;        /* GEMV output: qkv[conv_dim] | z[value_dim] | b[n_v] | a[n_v] */
    const float SGK_G *conv_w;    /* [conv_dim][ksize] */
    float SGK_G *ring;            /* [4][conv_dim] last inputs, slot = position % 4 */
    const float SGK_G *ssm_a;
    const float SGK_G *dt_bias;  /* [n_v] */
    float SGK_G *S;               /* [n_v][dv][dk] */
    float SGK_G *y;               /* [value_dim] */
    const sgk_step SGK_G *step;
    uint32_t n_k, n_v, dk, dv, conv_dim, ksize;
    int tiled, neg_exp;
    /* decode step only: z [value_dim] (the projection's z rows), norm_w the
     * ssm_norm weight [dv]; with blocks == 1 out receives RMSNormGated's
     * output, with SGK_GDN_BLOCKS out receives silu(z) * (y * norm_w) and ss
     * [n_v][SGK_GDN_BLOCKS] each row block's sum of squared readouts y, for
     * the gated GEMV prologue (y is not written) */
    const float SGK_G *z;
    const float SGK_G *norm_w;
    float SGK_G *out;
    float eps;
    float SGK_G *ss;
    uint32_t blocks;        /* workgroups per head: 1 (the step finishes RMSNormGated into out)
                             * or SGK_GDN_BLOCKS (out = silu(z), y and ss for the gated prologue) */
} sgk_gdn;
#define SGK_GDN_MAX_DV 256u
#define SGK_GDN_BLOCKS 4u
/* The decode step (blocks == 1: one workgroup per value head, dv <= 128;
 * else SGK_GDN_BLOCKS per head, dv <= SGK_GDN_MAX_DV, RMSNormGated's per-head
 * factor applied by the out projection's SGK_PRO_GATED prologue). */
hipError_t sgk_gdn_step(const sgk_gdn *a, hipStream_t s);

/* The DeltaNet layer over a prefill chunk of ntok tokens (a->step holds the
 * chunk's descriptors, a->in the chunk's GEMM rows at in_stride, a->y the
 * readouts [ntok][value_dim]): conv scan into conv_out [ntok][conv_dim], q/k
 * norms, then the delta-rule scan with S in registers. Same arithmetic as
 * sgk_gdn_step, token by token. */
hipError_t sgk_gdn_chunk(const sgk_gdn *a, float *conv_out, uint32_t in_stride, uint32_t ntok,
                         float *ws, hipStream_t s);
/* The delta-rule scan alone: qkv rows [ntok][a->conv_dim] hold normalised
 * q | k | v; gates [ntok][2*n_v] = beta | decay (or NULL: computed from the
 * b/a columns of a->in, rows in_stride apart, as in sgk_gdn_chunk). With a
 * workspace ws of sgk_delta_ws_floats(n_v, ntok) floats, dk 64 or 128 and
 * dv a multiple of 16 it runs the 16-token chunked form on the matrix cores;
 * with SURGE_DELTA_SCAN=seq, no workspace or other shapes the sequential
 * scan. */
hipError_t sgk_delta_scan(const sgk_gdn *a, const float *qkv, uint32_t in_stride, uint32_t ntok,
                          const float *gates, float *ws, hipStream_t s);
uint64_t sgk_delta_ws_floats(uint32_t n_v, uint32_t ntok);
/* Whether SURGE_DELTA_SCAN holds a form the scan knows (unset, empty, mfma,
 * seq); the host refuses to run with any other value. */
int sgk_delta_scan_env_ok(void);
/* Conv over a chunk with an oldest-first state [ksize-1][ch] in/out, no
 * activation (the reference's k_conv1d_chunk contract). */
hipError_t sgk_conv1d_chunk(const float *x, const float *w, float *out, float *state, uint32_t ch,
                            uint32_t ksize, uint32_t ntok, hipStream_t s);
/* beta/decay for every (token, head). */
hipError_t sgk_delta_gates_chunk(const float *a, const float *b, float *gates, const float *adt,
                                 uint32_t n, int neg_exp, uint32_t ntok, hipStream_t s);
/* silu(z) * rmsnorm(y, w) per (value head, token); z rows at z_stride. */
hipError_t sgk_rmsnorm_gated_rows(const float *y, const float *z, uint32_t z_stride, const float *w,
                                  float *out, uint32_t dv, uint32_t n_v, uint32_t ntok, float eps,
                                  hipStream_t s);
/* The same with the result written as the next prefill product's bf16 hi | lo
 * split of its X rows (sgk_gemm_args.xs layout, N = ntok, K = n_v*dv, which
 * must be a multiple of 32), for a product called with xs_ready. */
hipError_t sgk_rmsnorm_gated_split(const float *y, const float *z, uint32_t z_stride, const float *w,
                                   uint16_t *xs, uint32_t dv, uint32_t n_v, uint32_t ntok, float eps, hipStream_t s);
/* Embedding rows for a chunk: X[z] = row steps[z].token. */
hipError_t sgk_embed_rows(const int8_t *qs, const uint16_t *d, const float *wf, uint32_t hidden,
                          const sgk_step *steps, uint32_t ntok, float *X, hipStream_t s);

/* The bare delta rule over every value head (the per-op oracle hook):
 * qkv holds normalised q|k|v, gates = beta[n_v] | decay[n_v]. */
hipError_t sgk_delta_multi(float *S, const float *qkv, float *out, const float *gates,
                           uint32_t dk, uint32_t dv, uint32_t n_v, uint32_t n_k,
                           uint32_t key_dim, int tiled, hipStream_t s);
/* Single-token causal conv step (state oldest-first [ksize-1][channels]). */
hipError_t sgk_conv1d_step(const float *x, const float *w, float *y, float *state,
                           uint32_t channels, uint32_t ksize, hipStream_t s);
/* silu(z) * rmsnorm(y, w) per head of dv. */
hipError_t sgk_rmsnorm_gated(const float *y, const float *z, const float *w, float *out,
                             uint32_t dv, uint32_t heads, float eps, hipStream_t s);

/* Argmax over n floats, lowest index wins ties; result written to *out. */
hipError_t sgk_argmax(const float *v, uint32_t n, uint32_t *out, uint32_t *part,
                      hipStream_t s);

/* Greedy bookkeeping inside the decode graph: hist[pos + 1] = token (the
 * argmax just written into the descriptor), then pos += 1. */
hipError_t sgk_step_advance(sgk_step *step, uint32_t *hist, hipStream_t s);

/* Fills n f32 with a value (a kernel, so it may sit inside a captured graph). */
hipError_t sgk_fill_f32(float *p, float v, uint64_t n, hipStream_t s);
/* n seeded values in [-scale, scale], written as f16 bits (f16 != 0) or f32. */
hipError_t sgk_fill_hash(void *p, uint64_t n, int f16, uint32_t seed, float scale, hipStream_t s);

/* Prefill GEMM Y[N][M] = X[N][K] * W[M][K]^T with W in the Q8 device layout,
 * on MFMA (bf16 inputs, x split hi+lo, fp32 accumulate, per-block scale in
 * the accumulator). */
typedef struct {
    const float *X;          /* [N][ldx] */
    const int8_t *qs;        /* Q8 layout W [M][K] (or NULL with wf) */
    const uint16_t *dt;      /* its block scales, block-major [K/32][M] (sgk_repack_q8's dt) */
    const float *wf;         /* f32 W [M][K] */
    float *Y;                /* [N][ldy] */
    uint32_t N, M, K, ldx, ldy;
    int epi;                 /* SGK_EPI_*: store, += (residual), SwiGLU on (gate, up) column pairs */
    uint16_t *xs;            /* Q8 W: scratch of 2*N*K bf16, 16-byte aligned: X split into hi and lo,
                              * per Q8_0 block b and token n 32 hi then 32 lo at (b*N + n)*64 */
    float *part;             /* optional split-K partials (NULL: never split) */
    uint64_t part_cap;       /* floats in part */
    const float *nw;         /* Q8 W only: RMSNorm X's rows first (weight nw, eps), or NULL */
    float eps;
    int xs_ready;            /* Q8 W: xs already holds this product's split of X (with its RMSNorm) */
    const float *post_nw;    /* SGK_EPI_ADD, Q8 W, Y rows M wide: when the product splits K, its reduce also
                              * writes into xs the split of RMSNorm(Y rows) (weight post_nw, eps post_eps)
                              * that the next Q8 product over Y takes (xs must hold 2*N*M bf16), and sets
                              * *post_done (else 0) */
    float post_eps;
    int *post_done;
    uint16_t *ys;            /* SGK_EPI_SWIGLU, Q8 W: the SwiGLU outputs written as the next product's bf16
                              * split (the xs layout, N rows of M/2, (M/2) % 32 == 0) instead of into Y;
                              * must not alias xs */
} sgk_gemm_args;
/* Q8 W needs K % 32 == 0, ldx % 4 == 0 and X 16-byte aligned. */
hipError_t sgk_gemm(const sgk_gemm_args *a, hipStream_t s);
hipError_t sgk_gemm_q8(const float *X, const int8_t *qs, const uint16_t *dt, float *Y,
                       uint32_t N, uint32_t M, uint32_t K, uint16_t *xs, float *part,
                       uint64_t part_cap, hipStream_t s);

/* Widest rows the balanced GEMV (k_gemv_bal: one workgroup per CU, x staged
 * once) takes: columns a multiple of 1024, up to these. */
#define SGK_BAL_MAX_COLS 18432u
#define SGK_BAL_MAX_RMS_COLS 8192u         /* ... behind the RMSNorm prologue */
/* The device's compute units (the grid of one workgroup per CU). */
uint32_t sgk_device_cus(void);

/* Measurement kernels: a streaming read of `bytes` (a multiple of 16) by
 * `blocks` workgroups (one float per workgroup written to out), and an empty
 * kernel. */
hipError_t sgk_read(const void *p, uint64_t bytes, float *out, uint32_t blocks, hipStream_t s);
hipError_t sgk_empty(hipStream_t s);

/* The device-resident workspace of the no-allocation entry points: a
 * file-scope device array of SGK_SCRATCH_BYTES in kernels.hip. Call
 * sgk_scratch_init(dev) once per device with that device current; then
 * sgk_scratch_ptr(dev) is its device address (NULL before init). */
#define SGK_SCRATCH_BYTES (4u << 20)
hipError_t sgk_scratch_init(int dev);
void *sgk_scratch_ptr(int dev);

#ifdef __cplusplus
}
#endif
#endif
