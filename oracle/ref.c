/* oracle/ref.c - CPU oracle for the decode hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this file's library, and only as the checker or the timed CPU baseline.
 * The product library never links it; its GPU path fails loudly when its
 * own HIP code is missing rather than falling back to anything here.
 *
 * A from-scratch restatement of the reference's scalar CPU reference
 * (reference src/ref.c), written to reproduce its numbers bit for bit:
 *   - every reduction accumulates in double in strictly increasing index
 *     order, with the same association the reference uses;
 *   - transcendentals are libm's double-precision functions;
 *   - values are rounded to f32 at exactly the points the reference rounds.
 * Build with -ffp-contract=off so no multiply-add is fused (the reference's
 * own build does not fuse either: plain x86-64 has no FMA).
 *
 * Each function cites the reference lines it follows. Parity of this file is
 * pinned three ways in tests/test_oracle.py: against the reference's own
 * fixtures (ops.bin, hybrid_ops.bin, mini_fwd logits), against the reference
 * ref.c compiled from its sources into oracle/_ref (bit-exact), and against
 * closed forms and invariants.
 */
#include "ref.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int sg_ref_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ---------------------------------------------------------------------
 * Scalar conversions
 * --------------------------------------------------------------------- */

static float bits_to_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* bf16 is the top half of an f32 (ref.c:65-70). */
static float bf16_widen(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

/* Exact IEEE binary16 -> f32, subnormals included (ref.c:80-107). A
 * subnormal m * 2^-24 is rescaled as a double product, which is exact. */
float sg_ref_f16_to_f32(uint16_t h) {
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    float mag;
    if (e == 0) {
        mag = (float)ldexp((double)m, -24);             /* zero or subnormal */
    } else if (e == 31) {
        mag = bits_to_f32(0x7F800000u | (m << 13));     /* inf / nan payload */
    } else {
        mag = bits_to_f32(((e + 112u) << 23) | (m << 13));
    }
    return (h & 0x8000u) ? -mag : mag;
}

/* f32 -> binary16, round to nearest even; NaN -> quiet 0x7E00 with the sign
 * (kv.c:152-190). Works on the magnitude in units of the target's last place
 * so normal and subnormal results share one rounding step. */
uint16_t sg_ref_f32_to_f16(float f) {
    uint32_t x = f32_to_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* rounds past 65504 */
    int e = (int)(ax >> 23);                /* biased f32 exponent */
    uint32_t mant = (ax & 0x7FFFFFu) | (e ? 0x800000u : 0u);
    if (e == 0) e = 1;
    /* target unit: 2^-24 below 2^-14, else 2^(E-10) */
    int shift = (e < 113) ? (126 - e) : 13; /* bits to drop from the 24-bit mantissa */
    if (shift > 24) return sign;            /* < 2^-25: rounds to zero */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    if (e < 113) return (uint16_t)(sign | q);               /* subnormal (q may reach 0x400) */
    return (uint16_t)(sign | ((((uint32_t)(e - 112)) << 10) + (q - 0x400u)));
}

/* ---------------------------------------------------------------------
 * Elementwise and normalisation (ref.c:113-235)
 * --------------------------------------------------------------------- */

void sg_ref_rmsnorm(float *x, const float *w, uint32_t n, float eps) {
    if (!x || n == 0) return;
    double ss = 0.0;
    for (uint32_t i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    double r = 1.0 / sqrt(ss / (double)n + (double)eps);
    for (uint32_t i = 0; i < n; i++) {
        double v = (double)x[i] * r;
        x[i] = (float)(w ? v * (double)w[i] : v);
    }
}

float sg_ref_sigmoid(float x) {
    double d = x;
    if (d >= 0.0) return (float)(1.0 / (1.0 + exp(-d)));
    double e = exp(d);
    return (float)(e / (1.0 + e));
}

float sg_ref_softplus(float x) {
    double d = x;
    return (float)(fmax(d, 0.0) + log1p(exp(-fabs(d))));
}

float sg_ref_delta_decay(float a_log, float a, float dt_bias) {
    double g = exp((double)a_log) * (double)sg_ref_softplus(a + dt_bias);
    return (float)exp(-g);
}

float sg_ref_delta_decay_neg_a(float neg_a, float a, float dt_bias) {
    return (float)exp((double)neg_a * (double)sg_ref_softplus(a + dt_bias));
}

void sg_ref_silu(float *x, uint32_t n) {
    if (!x) return;
    for (uint32_t i = 0; i < n; i++) x[i] = (float)((double)x[i] * (double)sg_ref_sigmoid(x[i]));
}

void sg_ref_swiglu(float *gate, const float *up, uint32_t n) {
    if (!gate || !up) return;
    for (uint32_t i = 0; i < n; i++) {
        double a = (double)gate[i] * (double)sg_ref_sigmoid(gate[i]);
        gate[i] = (float)(a * (double)up[i]);
    }
}

void sg_ref_gate_sigmoid(float *x, const float *gate, uint32_t n) {
    if (!x || !gate) return;
    for (uint32_t i = 0; i < n; i++) x[i] = (float)((double)x[i] * (double)sg_ref_sigmoid(gate[i]));
}

void sg_ref_softmax(float *x, uint32_t n) {
    if (!x || n == 0) return;
    float mx = x[0];
    for (uint32_t i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    if (isnan(mx)) { for (uint32_t i = 0; i < n; i++) x[i] = mx; return; }
    if (isinf(mx)) {
        /* all -inf: uniform; any +inf: uniform over the +inf entries */
        uint32_t hits = 0;
        for (uint32_t i = 0; i < n; i++) hits += (x[i] == mx);
        float u = 1.0f / (float)(mx < 0 ? n : hits);
        for (uint32_t i = 0; i < n; i++) x[i] = (mx < 0 || x[i] == mx) ? u : 0.0f;
        return;
    }
    double sum = 0.0;
    for (uint32_t i = 0; i < n; i++) {
        double e = exp((double)x[i] - (double)mx);
        x[i] = (float)e;
        sum += e;
    }
    for (uint32_t i = 0; i < n; i++) x[i] = (float)((double)x[i] / sum);
}

/* ---------------------------------------------------------------------
 * Split-K combine and decode attention (ref.c:237-555)
 * --------------------------------------------------------------------- */

/* exp(mi - M), exactly 1 when the two are the same value (so +inf ties do not
 * become inf - inf) (ref.c:256-259). */
static double lse_weight(double mi, double M) { return mi == M ? 1.0 : exp(mi - M); }

void sg_ref_attn_combine(const float *m, const float *s, const float *acc,
                         uint32_t n_parts, uint32_t head_dim, float *out) {
    if (!out || head_dim == 0) return;
    if (n_parts > 0 && (!m || !s || !acc)) return;
    double M = n_parts ? (double)m[0] : -INFINITY;
    for (uint32_t i = 1; i < n_parts; i++) if ((double)m[i] > M) M = m[i];
    float fill = 0.0f;
    bool flat = false;
    if (n_parts == 0 || M == -INFINITY) { flat = true; }
    else if (isnan(M)) { flat = true; fill = (float)M; }
    double S = 0.0;
    if (!flat) {
        for (uint32_t i = 0; i < n_parts; i++) S += (double)s[i] * lse_weight(m[i], M);
        if (isnan(S)) { flat = true; fill = (float)S; }
    }
    if (flat) { for (uint32_t d = 0; d < head_dim; d++) out[d] = fill; return; }
    for (uint32_t d = 0; d < head_dim; d++) {
        double num = 0.0;
        for (uint32_t i = 0; i < n_parts; i++)
            num += (double)acc[(size_t)i * head_dim + d] * lse_weight(m[i], M);
        out[d] = S > 0.0 ? (float)(num / S) : 0.0f;
    }
}

/* One (head, key range) partial: two passes, each recomputing the score
 * (ref.c:416-455). Score is f32(double dot * double scale). */
static void partial_one(const float *qh, const float *kc, const float *vc,
                        uint32_t n_kv, uint32_t hk, uint32_t hd, double scale,
                        uint32_t t0, uint32_t t1, double *dacc,
                        float *m_out, float *s_out, float *acc_out) {
    if (t0 >= t1) {
        *m_out = -INFINITY;
        *s_out = 0.0f;
        memset(acc_out, 0, (size_t)hd * sizeof(float));
        return;
    }
    float mx = -INFINITY;
    for (uint32_t t = t0; t < t1; t++) {
        const float *kt = kc + ((size_t)t * n_kv + hk) * hd;
        double dot = 0.0;
        for (uint32_t i = 0; i < hd; i++) dot += (double)qh[i] * (double)kt[i];
        float sc = (float)(dot * scale);
        if (sc > mx) mx = sc;
    }
    double sum = 0.0;
    for (uint32_t d = 0; d < hd; d++) dacc[d] = 0.0;
    for (uint32_t t = t0; t < t1; t++) {
        const float *kt = kc + ((size_t)t * n_kv + hk) * hd;
        const float *vt = vc + ((size_t)t * n_kv + hk) * hd;
        double dot = 0.0;
        for (uint32_t i = 0; i < hd; i++) dot += (double)qh[i] * (double)kt[i];
        float sc = (float)(dot * scale);
        double e = exp((double)sc - (double)mx);
        sum += e;
        for (uint32_t d = 0; d < hd; d++) dacc[d] += e * (double)vt[d];
    }
    *m_out = mx;
    *s_out = (float)sum;
    for (uint32_t d = 0; d < hd; d++) acc_out[d] = (float)dacc[d];
}

/* Split i covers [i*seq/n, (i+1)*seq/n) in 64-bit arithmetic (ref.c:530-531). */
static uint32_t split_edge(uint32_t i, uint32_t seq, uint32_t n) {
    return (uint32_t)((uint64_t)i * seq / n);
}

void sg_ref_attn_partials(const float *q, const float *kc, const float *vc,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t seq, uint32_t q_stride, float scale,
                          uint32_t n_parts, float *m, float *s, float *acc) {
    if (!q || !kc || !vc || !m || !s || !acc || n_kv_heads == 0 || head_dim == 0) return;
    uint32_t rep = n_heads / n_kv_heads;
    double *dacc = malloc((size_t)head_dim * sizeof(double));
    if (!dacc) return;
    for (uint32_t h = 0; h < n_heads; h++) {
        uint32_t hk = rep ? h / rep : 0;
        for (uint32_t i = 0; i < n_parts; i++) {
            size_t o = (size_t)h * n_parts + i;
            partial_one(q + (size_t)h * q_stride, kc, vc, n_kv_heads, hk, head_dim,
                        (double)scale, split_edge(i, seq, n_parts),
                        split_edge(i + 1, seq, n_parts), dacc, &m[o], &s[o],
                        acc + o * head_dim);
        }
    }
    free(dacc);
}

/* Partitions, then one combine per head (ref.c:469-540). */
void sg_ref_attn_decode_splitk(const float *q, const float *kc, const float *vc,
                               uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                               uint32_t seq, uint32_t q_stride, float scale,
                               uint32_t n_parts, float *out) {
    if (!out || head_dim == 0 || n_heads == 0 || !q || !kc || !vc || n_kv_heads == 0) return;
    size_t np = n_parts ? n_parts : 1;
    float *m = malloc(np * sizeof(float)), *s = malloc(np * sizeof(float));
    float *acc = malloc(np * head_dim * sizeof(float));
    double *dacc = malloc((size_t)head_dim * sizeof(double));
    if (m && s && acc && dacc) {
        uint32_t rep = n_heads / n_kv_heads;
        for (uint32_t h = 0; h < n_heads; h++) {
            uint32_t hk = rep ? h / rep : 0;
            for (uint32_t i = 0; i < n_parts; i++)
                partial_one(q + (size_t)h * q_stride, kc, vc, n_kv_heads, hk, head_dim,
                            (double)scale, split_edge(i, seq, n_parts),
                            split_edge(i + 1, seq, n_parts), dacc, &m[i], &s[i],
                            acc + (size_t)i * head_dim);
            sg_ref_attn_combine(m, s, acc, n_parts, head_dim, out + (size_t)h * head_dim);
        }
    }
    free(m); free(s); free(acc); free(dacc);
}

void sg_ref_attn_decode(const float *q, const float *kc, const float *vc,
                        uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                        uint32_t seq, uint32_t q_stride, float scale, float *out) {
    sg_ref_attn_decode_splitk(q, kc, vc, n_heads, n_kv_heads, head_dim, seq, q_stride,
                              scale, 1, out);
}

/* ---------------------------------------------------------------------
 * RoPE (ref.c:561-606): half-split pairs, angle and sin/cos in double.
 * --------------------------------------------------------------------- */

void sg_ref_rope_partial(float *q, uint32_t head_dim, uint32_t rope_dim,
                         uint32_t pos, float theta) {
    if (!q || rope_dim < 2 || rope_dim > head_dim || (rope_dim & 1u)) return;
    uint32_t half = rope_dim / 2;
    for (uint32_t i = 0; i < half; i++) {
        double ang = (double)pos * pow((double)theta, -2.0 * (double)i / (double)rope_dim);
        double c = cos(ang), sn = sin(ang);
        double a = q[i], b = q[i + half];
        q[i] = (float)(a * c - b * sn);
        q[i + half] = (float)(a * sn + b * c);
    }
}

void sg_ref_rope(float *q, uint32_t head_dim, uint32_t pos, float theta) {
    sg_ref_rope_partial(q, head_dim, head_dim, pos, theta);
}

/* ---------------------------------------------------------------------
 * Matrix-vector products, y = W x, W row-major [rows, cols] (ref.c:612-663).
 * Rows are independent, so the OpenMP split changes no bit.
 * --------------------------------------------------------------------- */

void sg_ref_matvec_f32(const float *w, const float *x, float *y,
                       uint32_t rows, uint32_t cols) {
    if (!w || !x || !y) return;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const float *row = w + (size_t)r * cols;
        double acc = 0.0;
        for (uint32_t c = 0; c < cols; c++) acc += (double)row[c] * (double)x[c];
        y[r] = (float)acc;
    }
}

void sg_ref_matvec_bf16(const uint16_t *w, const float *x, float *y,
                        uint32_t rows, uint32_t cols) {
    if (!w || !x || !y) return;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const uint16_t *row = w + (size_t)r * cols;
        double acc = 0.0;
        for (uint32_t c = 0; c < cols; c++) acc += (double)bf16_widen(row[c]) * (double)x[c];
        y[r] = (float)acc;
    }
}

/* Q8_0 block: little-endian f16 scale (unaligned) then 32 int8. The block
 * dot is a double sum; the row sum adds d * block (ref.c:638-663). */
void sg_ref_matvec_q8(const void *w, const float *x, float *y,
                      uint32_t rows, uint32_t cols) {
    if (!w || !x || !y || cols % 32 != 0) return;
    const uint8_t *base = w;
    uint32_t nb = cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const uint8_t *blk = base + (size_t)r * nb * 34;
        double acc = 0.0;
        for (uint32_t b = 0; b < nb; b++, blk += 34) {
            double d = sg_ref_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            const int8_t *qs = (const int8_t *)(blk + 2);
            const float *xb = x + (size_t)b * 32;
            double part = 0.0;
            for (int i = 0; i < 32; i++) part += (double)qs[i] * (double)xb[i];
            acc += d * part;
        }
        y[r] = (float)acc;
    }
}

/* ---------------------------------------------------------------------
 * Gated DeltaNet primitives (ref.c:669-739)
 * --------------------------------------------------------------------- */

/* Depthwise causal conv over [carried state (oldest first), token]; tap
 * ksize-1 multiplies the newest token. In place on x; state_in may equal
 * state_out (each channel reads before it writes). */
void sg_ref_conv1d_causal(float *x, const float *w, const float *state_in,
                          float *state_out, uint32_t channels, uint32_t ksize) {
    if (!x || !w || ksize == 0 || channels == 0) return;
    uint32_t keep = ksize - 1;
    for (uint32_t c = 0; c < channels; c++) {
        const float *wc = w + (size_t)c * ksize;
        float cur = x[c];
        double acc = 0.0;
        if (state_in)
            for (uint32_t j = 0; j < keep; j++)
                acc += (double)wc[j] * (double)state_in[(size_t)j * channels + c];
        acc += (double)wc[keep] * (double)cur;
        if (state_out && keep) {
            for (uint32_t j = 0; j + 1 < keep; j++)
                state_out[(size_t)j * channels + c] =
                    state_in ? state_in[(size_t)(j + 1) * channels + c] : 0.0f;
            state_out[(size_t)(keep - 1) * channels + c] = cur;
        }
        x[c] = (float)acc;
    }
}

/* Per value row j: decay the row, read kv = row . k, delta = (v_j - kv) beta,
 * write row += k delta, read out_j = row . q from the updated row. */
void sg_ref_delta_step(float *S, const float *q, const float *k, const float *v,
                       float beta, float decay, float *out, uint32_t dk, uint32_t dv) {
    if (!S || !q || !k || !v || !out) return;
    for (uint32_t j = 0; j < dv; j++) {
        float *row = S + (size_t)j * dk;
        double kv = 0.0;
        for (uint32_t i = 0; i < dk; i++) {
            double sd = (double)row[i] * (double)decay;
            row[i] = (float)sd;
            kv += sd * (double)k[i];
        }
        double delta = ((double)v[j] - kv) * (double)beta;
        double y = 0.0;
        for (uint32_t i = 0; i < dk; i++) {
            double sn = (double)row[i] + (double)k[i] * delta;
            row[i] = (float)sn;
            y += sn * (double)q[i];
        }
        out[j] = (float)y;
    }
}

uint32_t sg_ref_argmax_f32(const float *v, uint32_t n) {
    if (!v || n == 0) return 0;
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}

/* =====================================================================
 * Whole-model forward (ref.c:741-1386)
 * ===================================================================== */

typedef struct {
    bool attn;
    float *kc, *vc;               /* [max_ctx, n_kv, hd] */
    float *conv, *S;              /* [ksize-1, conv_dim], [n_v, dv, dk] */
    float *ln1, *ln2, *qn, *kn, *ssm_norm, *conv_w, *dt_bias, *ssm_a;
} ref_layer;

struct sg_ref_state {
    const sg_model *owner;
    sg_cfg c;
    uint32_t max_ctx, used;
    uint32_t key_dim, value_dim, conv_dim, q_width, kv_width, attn_width;
    bool kv_f16;
    ref_layer *L;
    float *out_norm;
    float *x, *h, *r, *qg, *kb, *vb, *scores, *ctx, *gate;
    float *qkv, *z, *a, *b, *y, *ffg, *ffu, *logits;
    double *dacc;
};

static void mat(const sg_model *m, const void *w, const float *x, float *y,
                uint32_t rows, uint32_t cols) {
    if (m->wtype == SG_T_Q8_0) sg_ref_matvec_q8(w, x, y, rows, cols);
    else if (m->wtype == SG_T_BF16) sg_ref_matvec_bf16(w, x, y, rows, cols);
    else sg_ref_matvec_f32(w, x, y, rows, cols);
}

/* Small tensors widened once into owned f32, +shift for residual norms
 * (ref.c:789-809). */
static float *widen(const void *src, sg_tensor_type t, uint64_t n, float shift, bool *ok) {
    if (!*ok) return NULL;
    float *o = malloc((size_t)n * sizeof(float));
    if (!o) { *ok = false; return NULL; }
    for (uint64_t i = 0; i < n; i++)
        o[i] = (t == SG_T_BF16 ? bf16_widen(((const uint16_t *)src)[i])
                               : ((const float *)src)[i]) + shift;
    return o;
}

static float *zalloc(uint64_t n, bool *ok) {
    if (!*ok || n == 0) return NULL;
    float *p = calloc((size_t)n, sizeof(float));
    if (!p) *ok = false;
    return p;
}

/* Embedding row: Q8_0 is d * q in f32 (ref.c:826-854). */
static void embed_row(const sg_model *m, uint32_t tok, uint32_t hidden, float *out) {
    if (m->wtype == SG_T_Q8_0) {
        const uint8_t *p = (const uint8_t *)m->tok_emb + (size_t)tok * (hidden / 32) * 34;
        for (uint32_t b = 0; b < hidden / 32; b++, p += 34) {
            float d = sg_ref_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
            for (int i = 0; i < 32; i++) out[b * 32 + i] = d * (float)((const int8_t *)(p + 2))[i];
        }
    } else if (m->wtype == SG_T_BF16) {
        const uint16_t *p = (const uint16_t *)m->tok_emb + (size_t)tok * hidden;
        for (uint32_t i = 0; i < hidden; i++) out[i] = bf16_widen(p[i]);
    } else {
        memcpy(out, (const float *)m->tok_emb + (size_t)tok * hidden, hidden * sizeof(float));
    }
}

void sg_ref_state_free(sg_ref_state *st) {
    if (!st) return;
    if (st->L) {
        for (uint32_t i = 0; i < st->c.n_layers; i++) {
            ref_layer *L = &st->L[i];
            free(L->kc); free(L->vc); free(L->conv); free(L->S);
            free(L->ln1); free(L->ln2); free(L->qn); free(L->kn);
            free(L->ssm_norm); free(L->conv_w); free(L->dt_bias); free(L->ssm_a);
        }
        free(st->L);
    }
    float *bufs[] = { st->out_norm, st->x, st->h, st->r, st->qg, st->kb, st->vb,
                      st->scores, st->ctx, st->gate, st->qkv, st->z, st->a, st->b,
                      st->y, st->ffg, st->ffu, st->logits };
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; i++) free(bufs[i]);
    free(st->dacc);
    free(st);
}

void sg_ref_state_reset(sg_ref_state *st) {
    if (!st) return;
    st->used = 0;
    for (uint32_t i = 0; i < st->c.n_layers; i++) {
        ref_layer *L = &st->L[i];
        if (L->conv) memset(L->conv, 0, (size_t)(st->c.conv_kernel - 1) * st->conv_dim * 4);
        if (L->S) memset(L->S, 0, (size_t)st->c.n_v_heads * st->c.head_v_dim * st->c.head_k_dim * 4);
    }
}

void sg_ref_state_set_kv_f16(sg_ref_state *st, bool on) { if (st) st->kv_f16 = on; }

/* Test input, not part of the reference: the seeded decode state that the
 * product's sg_gpu_state_fill_synthetic writes (K/V rows [0, n) of every
 * attention layer, every DeltaNet S and conv tail), generated by the same
 * integer hash and the same f32 operations, so a decode step at depth can be
 * compared with the GPU's. Element i of a fill with seed s and scale c is
 * ((u0 + u1) - 1) * c with u0, u1 the low two 16-bit fields of
 * splitmix64((i + 1) * 0x9E3779B97F4A7C15 ^ (s << 32 | s)) divided by 65535;
 * K/V values are then rounded to f16. The GPU keeps K/V head-major and the
 * conv tail as a 4-slot ring indexed by position mod 4; this maps both onto
 * this state's layouts (K/V [pos][n_kv][hd]; conv tail oldest first, row j
 * taken from ring slot (n + 4 - (ksize-1) + j) mod 4). */
static float fill_val(uint64_t i, uint32_t seed, float scale) {
    uint64_t h = (i + 1) * 0x9E3779B97F4A7C15ull ^ ((uint64_t)seed << 32 | seed);
    h ^= h >> 31; h *= 0xBF58476D1CE4E5B9ull; h ^= h >> 29; h *= 0x94D049BB133111EBull; h ^= h >> 32;
    const float u0 = (float)(uint32_t)(h & 0xFFFFu) / 65535.0f, u1 = (float)(uint32_t)((h >> 16) & 0xFFFFu) / 65535.0f;
    return (u0 + u1 - 1.0f) * scale;
}

sg_err sg_ref_state_fill_synthetic(sg_ref_state *st, uint32_t n, uint32_t seed) {
    if (!st) return (sg_err){"ref: invalid arguments"};
    if (n >= st->max_ctx) return (sg_err){"ref: fill: n must be < max_ctx"};
    const sg_cfg *c = &st->c;
    const uint32_t nkv = c->n_kv_heads, hd = c->head_dim, cd = st->conv_dim, keep = c->conv_kernel - 1;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        ref_layer *L = &st->L[i];
        const uint32_t ls = seed * 2654435761u + 97u * i;
        if (L->attn) {
            for (uint32_t h = 0; h < nkv; h++)
                for (uint64_t e = 0; e < (uint64_t)n * hd; e++) {
                    const size_t at = ((size_t)(e / hd) * nkv + h) * hd + e % hd;
                    L->kc[at] = sg_ref_f16_to_f32(sg_ref_f32_to_f16(fill_val(e, ls + 2 * h, 2.0f)));
                    L->vc[at] = sg_ref_f16_to_f32(sg_ref_f32_to_f16(fill_val(e, ls + 2 * h + 1, 2.0f)));
                }
        } else {
            const uint64_t ns = (uint64_t)c->n_v_heads * c->head_v_dim * c->head_k_dim;
            for (uint64_t e = 0; e < ns; e++) L->S[e] = fill_val(e, ls + 7, 0.05f);
            for (uint32_t j = 0; j < keep; j++) {
                const uint32_t slot = (n + 4 - keep + j) & 3;
                for (uint32_t ch = 0; ch < cd; ch++)
                    L->conv[(size_t)j * cd + ch] = fill_val((uint64_t)slot * cd + ch, ls + 11, 0.05f);
            }
        }
    }
    st->used = n;
    return SG_OK;
}

/* Validation follows ref.c:965-1189: dims non-zero, layer kind by tensor
 * presence must agree with (L+1) % interval, rope/eps sanity, Q8_0 widths. */
sg_err sg_ref_state_new(const sg_model *m, uint32_t max_ctx, sg_ref_state **out) {
    if (!out) return (sg_err){"ref: invalid arguments"};
    *out = NULL;
    if (!m || !m->layers || !m->tok_emb || !m->out_norm || !m->lm_head)
        return (sg_err){"ref: invalid arguments"};
    const sg_cfg *c = &m->cfg;
    if (max_ctx == 0) return (sg_err){"ref: max_ctx must be at least 1"};
    if (!c->n_layers || !c->hidden || !c->ffn_hidden || !c->vocab || !c->head_dim ||
        !c->n_heads || !c->n_kv_heads)
        return (sg_err){"ref: model config has a zero dimension"};
    if (c->n_heads % c->n_kv_heads) return (sg_err){"ref: n_heads is not a multiple of n_kv_heads"};
    if (!c->full_attn_interval) return (sg_err){"ref: full_attn_interval is zero"};
    uint32_t n_attn = 0, n_gdn = 0;
    for (uint32_t i = 0; i < c->n_layers; i++) {
        bool is_attn = m->layers[i].q_proj != NULL;
        if (is_attn != ((i + 1) % c->full_attn_interval == 0))
            return (sg_err){"ref: layer kind disagrees with full_attn_interval"};
        n_attn += is_attn; n_gdn += !is_attn;
    }
    if (n_attn && (c->rope_dim < 2 || c->rope_dim > c->head_dim || (c->rope_dim & 1)))
        return (sg_err){"ref: rope_dim must be even and in [2, head_dim]"};
    if (n_attn && (!(c->rope_theta > 1.0f) || !isfinite(c->rope_theta)))
        return (sg_err){"ref: rope_theta must be finite and greater than 1"};
    if (!(c->rms_eps >= 0.0f) || !isfinite(c->rms_eps))
        return (sg_err){"ref: rms_eps must be finite and non-negative"};
    if (n_gdn && (!c->n_k_heads || !c->n_v_heads || !c->head_k_dim || !c->head_v_dim ||
                  !c->conv_kernel))
        return (sg_err){"ref: model has gated-DeltaNet layers but no DeltaNet dims"};
    if (n_gdn && c->n_v_heads % c->n_k_heads)
        return (sg_err){"ref: n_v_heads is not a multiple of n_k_heads"};

    sg_ref_state *st = calloc(1, sizeof *st);
    if (!st) return (sg_err){"ref: out of memory"};
    st->owner = m;
    st->c = *c;
    st->max_ctx = max_ctx;
    st->key_dim = c->n_k_heads * c->head_k_dim;
    st->value_dim = c->n_v_heads * c->head_v_dim;
    st->conv_dim = 2 * st->key_dim + st->value_dim;
    st->attn_width = c->n_heads * c->head_dim;
    st->q_width = c->attn_output_gate ? 2 * st->attn_width : st->attn_width;
    st->kv_width = c->n_kv_heads * c->head_dim;
    if (m->wtype == SG_T_Q8_0) {
        uint32_t w[] = { c->hidden, c->ffn_hidden, st->attn_width, st->value_dim };
        for (int i = 0; i < 4; i++)
            if (w[i] % 32) { free(st); return (sg_err){"ref: a Q8_0 matmul width is not a multiple of 32"}; }
    }
    bool ok = true;
    st->L = calloc(c->n_layers, sizeof *st->L);
    if (!st->L) ok = false;
    float sh = m->norms_are_residual ? 1.0f : 0.0f;
    st->out_norm = widen(m->out_norm, m->dense_type, c->hidden, sh, &ok);
    st->x = zalloc(c->hidden, &ok); st->h = zalloc(c->hidden, &ok); st->r = zalloc(c->hidden, &ok);
    st->ffg = zalloc(c->ffn_hidden, &ok); st->ffu = zalloc(c->ffn_hidden, &ok);
    st->logits = zalloc(c->vocab, &ok);
    st->dacc = ok ? calloc(c->head_dim, sizeof(double)) : NULL;
    if (!st->dacc) ok = false;
    if (n_attn) {
        st->qg = zalloc(st->q_width, &ok); st->kb = zalloc(st->kv_width, &ok);
        st->vb = zalloc(st->kv_width, &ok); st->scores = zalloc(max_ctx, &ok);
        st->ctx = zalloc(st->attn_width, &ok); st->gate = zalloc(st->attn_width, &ok);
    }
    if (n_gdn) {
        st->qkv = zalloc(st->conv_dim, &ok); st->z = zalloc(st->value_dim, &ok);
        st->a = zalloc(c->n_v_heads, &ok); st->b = zalloc(c->n_v_heads, &ok);
        st->y = zalloc(st->value_dim, &ok);
    }
    for (uint32_t i = 0; ok && i < c->n_layers; i++) {
        const sg_layer_w *w = &m->layers[i];
        ref_layer *L = &st->L[i];
        L->attn = w->q_proj != NULL;
        L->ln1 = widen(w->ln1, m->dense_type, c->hidden, sh, &ok);
        L->ln2 = widen(w->ln2, m->dense_type, c->hidden, sh, &ok);
        if (L->attn) {
            L->qn = widen(w->q_norm, m->dense_type, c->head_dim, sh, &ok);
            L->kn = widen(w->k_norm, m->dense_type, c->head_dim, sh, &ok);
            L->kc = zalloc((uint64_t)max_ctx * st->kv_width, &ok);
            L->vc = zalloc((uint64_t)max_ctx * st->kv_width, &ok);
        } else {
            L->ssm_norm = widen(w->ssm_norm, m->ssm_norm_type, c->head_v_dim, 0.0f, &ok);
            L->ssm_a = widen(w->ssm_a, m->ssm_a_type, c->n_v_heads, 0.0f, &ok);
            L->conv_w = widen(w->ssm_conv1d, m->dense_type,
                              (uint64_t)st->conv_dim * c->conv_kernel, 0.0f, &ok);
            L->dt_bias = widen(w->ssm_dt_bias, m->dense_type, c->n_v_heads, 0.0f, &ok);
            L->conv = zalloc((uint64_t)(c->conv_kernel - 1) * st->conv_dim, &ok);
            L->S = zalloc((uint64_t)c->n_v_heads * c->head_v_dim * c->head_k_dim, &ok);
        }
    }
    if (!ok) { sg_ref_state_free(st); return (sg_err){"ref: out of memory"}; }
    *out = st;
    return SG_OK;
}

static float kv_round(const sg_ref_state *st, float v) {
    return st->kv_f16 ? sg_ref_f16_to_f32(sg_ref_f32_to_f16(v)) : v;
}

/* Full attention for one token (ref.c:1197-1269). */
static void attn_mixer(sg_ref_state *st, const sg_model *m, const sg_layer_w *w,
                       ref_layer *L, uint32_t pos) {
    const sg_cfg *c = &st->c;
    uint32_t hd = c->head_dim, qs = c->attn_output_gate ? 2 * hd : hd;
    mat(m, w->q_proj, st->h, st->qg, st->q_width, c->hidden);
    mat(m, w->k_proj, st->h, st->kb, st->kv_width, c->hidden);
    mat(m, w->v_proj, st->h, st->vb, st->kv_width, c->hidden);
    for (uint32_t h = 0; h < c->n_heads; h++) {
        float *qh = st->qg + (size_t)h * qs;
        sg_ref_rmsnorm(qh, L->qn, hd, c->rms_eps);
        sg_ref_rope_partial(qh, hd, c->rope_dim, pos, c->rope_theta);
        if (c->attn_output_gate) memcpy(st->gate + (size_t)h * hd, qh + hd, hd * sizeof(float));
    }
    for (uint32_t h = 0; h < c->n_kv_heads; h++) {
        float *kh = st->kb + (size_t)h * hd;
        sg_ref_rmsnorm(kh, L->kn, hd, c->rms_eps);
        sg_ref_rope_partial(kh, hd, c->rope_dim, pos, c->rope_theta);
    }
    float *kd = L->kc + (size_t)pos * st->kv_width, *vd = L->vc + (size_t)pos * st->kv_width;
    for (uint32_t i = 0; i < st->kv_width; i++) {
        kd[i] = kv_round(st, st->kb[i]);
        vd[i] = kv_round(st, st->vb[i]);
    }
    uint32_t n = pos + 1, rep = c->n_heads / c->n_kv_heads;
    double scale = 1.0 / sqrt((double)hd);
    for (uint32_t h = 0; h < c->n_heads; h++) {
        uint32_t hk = h / rep;
        const float *qh = st->qg + (size_t)h * qs;
        for (uint32_t t = 0; t < n; t++) {
            const float *kt = L->kc + ((size_t)t * c->n_kv_heads + hk) * hd;
            double dot = 0.0;
            for (uint32_t i = 0; i < hd; i++) dot += (double)qh[i] * (double)kt[i];
            st->scores[t] = (float)(dot * scale);
        }
        sg_ref_softmax(st->scores, n);
        for (uint32_t i = 0; i < hd; i++) st->dacc[i] = 0.0;
        for (uint32_t t = 0; t < n; t++) {
            const float *vt = L->vc + ((size_t)t * c->n_kv_heads + hk) * hd;
            double p = st->scores[t];
            for (uint32_t i = 0; i < hd; i++) st->dacc[i] += p * (double)vt[i];
        }
        for (uint32_t i = 0; i < hd; i++) st->ctx[(size_t)h * hd + i] = (float)st->dacc[i];
    }
    if (c->attn_output_gate) sg_ref_gate_sigmoid(st->ctx, st->gate, st->attn_width);
    mat(m, w->o_proj, st->ctx, st->r, c->hidden, st->attn_width);
}

/* Gated DeltaNet for one token (ref.c:1273-1333). */
static void gdn_mixer(sg_ref_state *st, const sg_model *m, const sg_layer_w *w, ref_layer *L) {
    const sg_cfg *c = &st->c;
    uint32_t dk = c->head_k_dim, dv = c->head_v_dim;
    mat(m, w->ssm_in_qkv, st->h, st->qkv, st->conv_dim, c->hidden);
    mat(m, w->ssm_in_z, st->h, st->z, st->value_dim, c->hidden);
    mat(m, w->ssm_in_b, st->h, st->b, c->n_v_heads, c->hidden);
    mat(m, w->ssm_in_a, st->h, st->a, c->n_v_heads, c->hidden);
    sg_ref_conv1d_causal(st->qkv, L->conv_w, L->conv, L->conv, st->conv_dim, c->conv_kernel);
    sg_ref_silu(st->qkv, st->conv_dim);
    float *q = st->qkv, *k = st->qkv + st->key_dim, *v = st->qkv + 2 * st->key_dim;
    double inv = 1.0 / sqrt((double)dk);
    for (uint32_t h = 0; h < c->n_k_heads; h++) {
        float *qh = q + (size_t)h * dk, *kh = k + (size_t)h * dk;
        sg_ref_rmsnorm(qh, NULL, dk, 1e-6f);
        sg_ref_rmsnorm(kh, NULL, dk, 1e-6f);
        for (uint32_t i = 0; i < dk; i++) {
            qh[i] = (float)((double)qh[i] * inv * inv);
            kh[i] = (float)((double)kh[i] * inv);
        }
    }
    for (uint32_t h = 0; h < c->n_v_heads; h++) {
        uint32_t hk = sg_ssm_k_head(h, c->n_k_heads, c->n_v_heads, m->v_heads_tiled);
        float beta = sg_ref_sigmoid(st->b[h]);
        float decay = m->ssm_a_form == SG_SSM_A_NEG_EXP
                          ? sg_ref_delta_decay_neg_a(L->ssm_a[h], st->a[h], L->dt_bias[h])
                          : sg_ref_delta_decay(L->ssm_a[h], st->a[h], L->dt_bias[h]);
        sg_ref_delta_step(L->S + (size_t)h * dv * dk, q + (size_t)hk * dk, k + (size_t)hk * dk,
                          v + (size_t)h * dv, beta, decay, st->y + (size_t)h * dv, dk, dv);
    }
    for (uint32_t h = 0; h < c->n_v_heads; h++) {
        float *yh = st->y + (size_t)h * dv, *zh = st->z + (size_t)h * dv;
        sg_ref_rmsnorm(yh, L->ssm_norm, dv, c->rms_eps);
        sg_ref_swiglu(zh, yh, dv);
        memcpy(yh, zh, dv * sizeof(float));
    }
    mat(m, w->ssm_out, st->y, st->r, c->hidden, st->value_dim);
}

sg_err sg_ref_forward(sg_ref_state *st, const sg_model *m, int32_t token,
                      uint32_t pos, const float **logits) {
    if (!st || !m || !m->layers) return (sg_err){"ref: invalid arguments"};
    if (m != st->owner) return (sg_err){"ref: this state was built for a different sg_model"};
    const sg_cfg *c = &st->c;
    if (token < 0 || (uint32_t)token >= c->vocab) return (sg_err){"ref: token id out of range"};
    if (pos >= st->max_ctx) return (sg_err){"ref: position exceeds max_ctx"};
    if (pos != st->used) return (sg_err){"ref: positions must be presented in order"};
    embed_row(m, (uint32_t)token, c->hidden, st->x);
    for (uint32_t i = 0; i < c->n_layers; i++) {
        const sg_layer_w *w = &m->layers[i];
        ref_layer *L = &st->L[i];
        memcpy(st->h, st->x, c->hidden * sizeof(float));
        sg_ref_rmsnorm(st->h, L->ln1, c->hidden, c->rms_eps);
        if (L->attn) attn_mixer(st, m, w, L, pos); else gdn_mixer(st, m, w, L);
        for (uint32_t j = 0; j < c->hidden; j++) st->x[j] += st->r[j];
        memcpy(st->h, st->x, c->hidden * sizeof(float));
        sg_ref_rmsnorm(st->h, L->ln2, c->hidden, c->rms_eps);
        mat(m, w->gate_proj, st->h, st->ffg, c->ffn_hidden, c->hidden);
        mat(m, w->up_proj, st->h, st->ffu, c->ffn_hidden, c->hidden);
        sg_ref_swiglu(st->ffg, st->ffu, c->ffn_hidden);
        mat(m, w->down_proj, st->ffg, st->r, c->hidden, c->ffn_hidden);
        for (uint32_t j = 0; j < c->hidden; j++) st->x[j] += st->r[j];
    }
    memcpy(st->h, st->x, c->hidden * sizeof(float));
    sg_ref_rmsnorm(st->h, st->out_norm, c->hidden, c->rms_eps);
    mat(m, m->lm_head, st->h, st->logits, c->vocab, c->hidden);
    st->used = pos + 1;
    if (logits) *logits = st->logits;
    return SG_OK;
}
